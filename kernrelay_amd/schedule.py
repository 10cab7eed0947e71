"""DAG model and fixed row-split schedules consumed by kr_plan_run.

Behaviour follows the reference's scheduler for this path:

* ``build_fixed_schedule`` — python/kernrelay/_vendor/scheduler/fixed.py:64-156:
  every node's input rows are split evenly into its chunk count; consumer
  tile j waits on every producer tile whose output rows intersect j's input
  rows (the last producer tile when none do); waits are only materialised
  across streams; tasks enter their stream in DAG topological order
  (declaration order breaks ties);
* ``serial_schedule`` — python/kernrelay/schedule.py:67-105: all tiles on one
  ``aicore`` stream in a global topological order, no waits or publishes;
* ``validate_schedule`` / ``invalid_variants`` — python/kernrelay/schedule.py:
  108-222: the structural checks and the four deliberately broken schedules
  whose executor error markers the E0 gate expects.

Op -> stream follows the reference's measured engine map
(python/kernrelay/_vendor/registry/engine_map.json): matrix work on ``aic``,
vector work on ``aiv``. On MI355X ``aic`` is the producer HIP stream and
``aiv`` the consumer stream of the relay. The MI355X build adds the Qwen
relay consumers (silu, mul, swiglu, rmsnorm, add_rmsnorm) as ``aiv`` ops and
lets a node carry ``dtype`` (fp16 | bf16), ``to`` (cast target), ``eps`` and
``inputs`` (files replacing the deterministic inputs).
"""

import copy
import json
from dataclasses import dataclass, field
from pathlib import Path

ENGINES = ("aicore", "aic", "aiv", "aicpu", "hccl")

STREAM_OF_OP = {
    "matmul": "aic",
    "add": "aiv", "gelu": "aiv", "softmax": "aiv", "layernorm": "aiv", "cast": "aiv",
    "silu": "aiv", "mul": "aiv", "swiglu": "aiv", "rmsnorm": "aiv", "add_rmsnorm": "aiv",
    "embedding": "aiv",
    "topk": "aicore", "sort": "aicore",
    "allreduce": "hccl", "allgather": "hccl", "reducescatter": "hccl",
}

SHAPE_KEYS = {"matmul": ("M", "K", "N"), "topk": ("rows", "cols", "k"),
              "embedding": ("rows", "cols", "vocab")}

EXTRA_KEYS = ("inputs", "to", "eps")


def stream_of(op):
    """Physical stream of an op; unknown ops are treated as MIX (``aicore``)."""
    return STREAM_OF_OP.get(op, "aicore")


@dataclass
class Node:
    name: str
    op: str
    engine: str
    shape: dict
    dtype: str = "fp16"
    tiles: int = 1
    extra: dict = field(default_factory=dict)


@dataclass
class Edge:
    src: str
    dst: str
    kind: str = "data"


@dataclass
class Dag:
    name: str
    description: str = ""
    nodes: list = field(default_factory=list)
    edges: list = field(default_factory=list)

    @property
    def node_map(self):
        return {n.name: n for n in self.nodes}

    def validate(self):
        names = [n.name for n in self.nodes]
        if len(names) != len(set(names)):
            raise ValueError("%s: duplicate node names" % self.name)
        nm = self.node_map
        for n in self.nodes:
            if n.engine not in ENGINES:
                raise ValueError("%s: node %s has unknown engine %s" % (self.name, n.name, n.engine))
            if n.tiles < 1:
                raise ValueError("%s: node %s needs tiles >= 1" % (self.name, n.name))
            for k in SHAPE_KEYS.get(n.op, ("rows", "cols")):
                if k not in n.shape:
                    raise ValueError("%s: node %s shape lacks %s" % (self.name, n.name, k))
                if int(n.shape[k]) <= 0:
                    raise ValueError("%s: node %s shape[%s] must be > 0" % (self.name, n.name, k))
        keys = [(e.src, e.dst) for e in self.edges]
        if len(keys) != len(set(keys)):
            raise ValueError("%s: duplicate edges" % self.name)
        for e in self.edges:
            if e.src not in nm or e.dst not in nm:
                raise ValueError("%s: edge %s->%s names an unknown node" % (self.name, e.src, e.dst))
            if e.src == e.dst:
                raise ValueError("%s: self edge %s" % (self.name, e.src))
        return self


def dag_from_dict(raw):
    nodes = []
    for n in raw["nodes"]:
        extra = {k: n[k] for k in EXTRA_KEYS if k in n}
        nodes.append(Node(n["name"], n["op"], n.get("engine", stream_of(n["op"])), dict(n["shape"]),
                          n.get("dtype", "fp16"), int(n.get("tiles", 1)), extra))
    edges = [Edge(e["src"], e["dst"], e.get("kind", "data")) for e in raw["edges"]]
    return Dag(raw["name"], raw.get("description", ""), nodes, edges).validate()


def load_dag(path):
    """DAG JSON file -> Dag (the reference's dags/*.json format)."""
    return dag_from_dict(json.loads(Path(path).read_text(encoding="utf-8")))


def load_fixed_dag(path):
    """(Dag, fixed chunking) from a DAG file's optional ``fixed.chunking``."""
    raw = json.loads(Path(path).read_text(encoding="utf-8"))
    dag = dag_from_dict(raw)
    chunking = dict((raw.get("fixed") or {}).get("chunking") or {})
    unknown = set(chunking) - {n.name for n in dag.nodes}
    if unknown:
        raise ValueError("%s: fixed.chunking names unknown nodes %s" % (dag.name, sorted(unknown)))
    return dag, chunking


def node_rows(node):
    """Input rows of a node (M for matmul)."""
    return int(node.shape["M"]) if node.op == "matmul" else int(node.shape["rows"])


def out_rows(node, nranks):
    """Output rows; collectives scale them (allgather x nranks, reducescatter / nranks)."""
    rows = node_rows(node)
    if node.op == "allgather":
        return rows * nranks
    if node.op == "reducescatter":
        return rows // nranks
    return rows


def node_dims(node):
    """DAG shape -> executor fields (rows/cols/k/n/dim0)."""
    s = node.shape
    if node.op == "matmul":
        return {"rows": int(s["M"]), "cols": int(s["N"]), "k": int(s["K"]), "n": int(s["N"])}
    if node.op == "topk":
        return {"rows": int(s["rows"]), "cols": int(s["cols"]), "k": int(s["k"])}
    if node.op == "embedding":
        return {"rows": int(s["rows"]), "cols": int(s["cols"]), "dim0": int(s["vocab"])}
    return {"rows": int(s["rows"]), "cols": int(s["cols"])}


def topo_order(dag):
    """Kahn order; among ready nodes the earliest declared goes first."""
    names = [n.name for n in dag.nodes]
    pos = {n: i for i, n in enumerate(names)}
    indeg = {n: 0 for n in names}
    succ = {n: [] for n in names}
    for e in dag.edges:
        indeg[e.dst] += 1
        succ[e.src].append(e.dst)
    ready = sorted((n for n in names if indeg[n] == 0), key=pos.get)
    order = []
    while ready:
        cur = ready.pop(0)
        order.append(cur)
        for v in succ[cur]:
            indeg[v] -= 1
            if indeg[v] == 0:
                ready.append(v)
                ready.sort(key=pos.get)
    if len(order) != len(names):
        raise ValueError("%s: the DAG has a cycle" % dag.name)
    return order


def build_fixed_schedule(dag, chunking=None, nranks=1, method="fixed"):
    """DAG + fixed chunking -> schedule.json content (dict)."""
    chunking = {k: int(v) for k, v in dict(chunking or {}).items() if int(v) > 0}
    nm = dag.node_map
    unknown = set(chunking) - set(nm)
    if unknown:
        raise ValueError("%s: chunking names unknown nodes %s" % (dag.name, sorted(unknown)))
    for e in dag.edges:
        if nm[e.src].op == "cast":
            raise ValueError("%s: a cast output may only be a sink, not consumed by %s" % (dag.name, e.dst))

    geom = {}
    for n in dag.nodes:
        rows = node_rows(n)
        chunks = chunking.get(n.name, 1)
        if rows % chunks != 0:
            raise ValueError("%s: node %s rows=%d not divisible by chunks=%d" % (dag.name, n.name, rows, chunks))
        own_out = out_rows(n, nranks)
        if own_out % chunks != 0:
            raise ValueError("%s: node %s output rows %d not divisible by chunks=%d"
                             % (dag.name, n.name, own_out, chunks))
        if n.op == "reducescatter" and (rows // chunks) % nranks != 0:
            raise ValueError("%s: reducescatter %s rows per chunk must divide by nranks=%d"
                             % (dag.name, n.name, nranks))
        geom[n.name] = (chunks, rows // chunks, own_out // chunks)

    tasks = {}
    for n in dag.nodes:
        chunks, per, out_per = geom[n.name]
        for i in range(chunks):
            tasks[(n.name, i)] = {"node": n.name, "tile": i, "wait": [], "publish": False,
                                  "in_row_off": i * per, "in_rows": per, "out_row_off": i * out_per}

    published = set()
    for e in dag.edges:
        src, dst = nm[e.src], nm[e.dst]
        src_chunks, _, src_out_per = geom[src.name]
        dst_chunks, dst_per, _ = geom[dst.name]
        src_out = out_rows(src, nranks)
        if node_rows(dst) > src_out:
            raise ValueError("%s: edge %s->%s consumer reads %d rows but the producer writes %d"
                             % (dag.name, e.src, e.dst, node_rows(dst), src_out))
        if stream_of(src.op) == stream_of(dst.op):
            continue  # same stream: FIFO order already serialises them
        for j in range(dst_chunks):
            lo, hi = j * dst_per, (j + 1) * dst_per
            hits = [k for k in range(src_chunks) if k * src_out_per < hi and (k + 1) * src_out_per > lo]
            if not hits:
                hits = [src_chunks - 1]
            for k in hits:
                if k * src_out_per >= src_out:
                    continue
                tasks[(dst.name, j)]["wait"].append([src.name, k])
                published.add((src.name, k))
    for key in published:
        tasks[key]["publish"] = True

    streams = {}
    for name in topo_order(dag):
        s = stream_of(nm[name].op)
        for i in range(geom[name][0]):
            streams.setdefault(s, []).append(tasks[(name, i)])

    nodes = []
    for n in dag.nodes:
        entry = {"id": n.name, "op": n.op, "engine": stream_of(n.op), "dtype": n.dtype,
                 "tiles": geom[n.name][0], "split": geom[n.name][0] > 1,
                 "preds": [e.src for e in dag.edges if e.dst == n.name], "iters": 1, "blocks": 1}
        entry.update(node_dims(n))
        entry.update(n.extra)
        nodes.append(entry)
    return {"dag": dag.name, "group": method, "nranks": int(nranks), "nodes": nodes,
            "streams": {k: v for k, v in streams.items() if v},
            "chunking": {k: v for k, v in chunking.items() if v > 1}, "fallback": ""}


def serial_schedule(dag, nranks=1):
    """Serial baseline: every tile on one ``aicore`` stream in topological order."""
    base = build_fixed_schedule(dag, {}, nranks=nranks, method="serial")
    order = {"aicore": 0, "compute": 0, "aic": 1, "aiv": 2, "aicpu": 3, "hccl": 4}
    tasks, rank, deps = {}, {}, {}
    for engine, seq in base["streams"].items():
        for i, t in enumerate(seq):
            key = (t["node"], int(t.get("tile", 0)))
            tasks[key] = t
            rank[key] = (order.get(engine, 9), i)
    for engine, seq in base["streams"].items():
        for i, t in enumerate(seq):
            key = (t["node"], int(t.get("tile", 0)))
            d = {(w[0], int(w[1])) for w in (t.get("wait") or [])}
            if i:
                p = seq[i - 1]
                d.add((p["node"], int(p.get("tile", 0))))
            deps[key] = {x for x in d if x in tasks}
    done, ordered = set(), []
    while len(ordered) < len(tasks):
        ready = [k for k in tasks if k not in done and deps[k] <= done]
        if not ready:
            raise RuntimeError("%s: serial baseline has a cycle" % dag.name)
        key = min(ready, key=lambda k: rank[k])
        ordered.append(key)
        done.add(key)
    merged = []
    for key in ordered:
        t = dict(tasks[key])
        t["wait"] = []
        t["publish"] = False
        merged.append(t)
    out = dict(base)
    out["streams"] = {"aicore": merged}
    out["group"] = "serial"
    out["chunking"] = {}
    return out


def validate_schedule(sched):
    """Structural checks (the executor stays the authority). Returns errors."""
    errors = []
    nodes = sched.get("nodes") or []
    ids = [n.get("id") for n in nodes]
    if len(ids) != len(set(ids)):
        errors.append("duplicate node ids")
    known = set(ids)
    streams = sched.get("streams") or {}
    if not streams:
        errors.append("no streams")
    items, seen = [], {}
    for engine, seq in streams.items():
        if engine not in ENGINES:
            errors.append("unknown stream %r" % engine)
        if not isinstance(seq, list):
            errors.append("stream %r is not a task list" % engine)
            continue
        for i, t in enumerate(seq):
            key = (t.get("node"), int(t.get("tile", 0)))
            if key[0] not in known:
                errors.append("stream %s task names unknown node %r" % (engine, key[0]))
            if key in seen:
                errors.append("node %s tile %d repeated on streams %s/%s" % (key[0], key[1], seen[key], engine))
            seen[key] = engine
            if int(t.get("in_rows", 1)) <= 0:
                errors.append("node %s tile %d has in_rows <= 0" % key)
            items.append((key, engine, t))
    published = {(t.get("node"), int(t.get("tile", 0))) for seq in streams.values() for t in seq
                 if t.get("publish")}
    pos = {item[0]: i for i, item in enumerate(items)}
    adj = {i: set() for i in range(len(items))}
    indeg = {i: 0 for i in range(len(items))}
    last = {}
    for i, (_, engine, _) in enumerate(items):
        if engine in last:
            adj[last[engine]].add(i)
            indeg[i] += 1
        last[engine] = i
    for i, (key, _, t) in enumerate(items):
        for w in t.get("wait") or []:
            wkey = (w[0], int(w[1]))
            if wkey not in pos:
                errors.append("node %s tile %d waits on missing task %s#%s" % (key[0], key[1], wkey[0], wkey[1]))
                continue
            if wkey not in published:
                errors.append("node %s tile %d waits on %s#%s which never publishes"
                              % (key[0], key[1], wkey[0], wkey[1]))
            j = pos[wkey]
            if i not in adj[j]:
                adj[j].add(i)
                indeg[i] += 1
    ready = [i for i, d in indeg.items() if d == 0]
    done = 0
    while ready:
        cur = ready.pop()
        done += 1
        for nxt in adj[cur]:
            indeg[nxt] -= 1
            if indeg[nxt] == 0:
                ready.append(nxt)
    if done != len(items):
        errors.append("schedule has a wait cycle")
    return errors


def invalid_variants(sched):
    """Deterministic broken copies of a schedule and the executor error
    marker each must produce (reference python/kernrelay/schedule.py:185-222)."""
    out = {}
    dup = copy.deepcopy(sched)
    first = next(k for k in dup["streams"] if dup["streams"][k])
    dup["streams"]["compute"] = dup["streams"].pop(first)
    dup["streams"]["aicore"] = []
    out["duplicate_engine"] = (dup, "duplicate engine stream")

    ghost = copy.deepcopy(sched)
    first = next(k for k, v in ghost["streams"].items() if v)
    ghost["streams"][first].append({"node": "__ghost__", "tile": 0, "wait": [], "publish": False,
                                    "in_row_off": 0, "in_rows": 1})
    out["ghost_task"] = (ghost, "missing plan for task")

    cycle = copy.deepcopy(sched)
    names = [k for k, v in cycle["streams"].items() if v]
    if len(names) < 2:
        return out
    t0 = cycle["streams"][names[0]][0]
    t1 = cycle["streams"][names[1]][0]
    t0["publish"] = True
    t1["publish"] = True
    t0.setdefault("wait", []).append([t1["node"], int(t1.get("tile", 0))])
    t1.setdefault("wait", []).append([t0["node"], int(t0.get("tile", 0))])
    out["wait_cycle"] = (cycle, "wait cycle")

    over = copy.deepcopy(sched)
    for seq in over["streams"].values():
        for t in seq:
            if t.get("in_row_off", 0) > 0:
                t["in_rows"] = int(t["in_rows"]) + 10 ** 9
                out["row_overflow"] = (over, "exceed")
                return out
    return out


def dump_schedule(sched, path):
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(sched, indent=1), encoding="utf-8")
    return path
