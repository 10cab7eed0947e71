"""DAG model and fixed row-split schedules consumed by kr_plan_run.

Behaviour follows the reference's scheduler for this path:

* ``build_fixed_schedule`` — the schedule.json the reference's fixed-plan
  writer emits (python/kernrelay/_vendor/scheduler/fixed.py:64-156): every
  node's input rows are split evenly into its chunk count; consumer tile j
  waits on every producer tile whose output rows meet j's input rows (the
  last producer tile when none do); waits exist only across streams; tasks
  enter their stream in DAG topological order (declaration order breaks
  ties);
* ``serial_schedule`` — the reference's serial baseline
  (python/kernrelay/schedule.py:67-105): all tiles on one ``aicore`` stream
  in a global topological order, no waits or publishes;
* ``validate_schedule`` / ``invalid_variants`` — structural checks, and the
  four deliberately broken schedules whose executor error markers the
  reference's E0 gate expects (python/kernrelay/schedule.py:108-222).

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
    """Node names in dependency order; of the nodes whose producers are all
    placed, the one declared first goes next (a min-heap on declaration
    index)."""
    import heapq
    index = {n.name: i for i, n in enumerate(dag.nodes)}
    waiting = {n.name: 0 for n in dag.nodes}
    consumers = {n.name: [] for n in dag.nodes}
    for e in dag.edges:
        waiting[e.dst] += 1
        consumers[e.src].append(e.dst)
    heap = [index[name] for name, w in waiting.items() if w == 0]
    heapq.heapify(heap)
    order = []
    while heap:
        name = dag.nodes[heapq.heappop(heap)].name
        order.append(name)
        for c in consumers[name]:
            waiting[c] -= 1
            if waiting[c] == 0:
                heapq.heappush(heap, index[c])
    if len(order) != len(dag.nodes):
        raise ValueError("%s: the DAG has a cycle" % dag.name)
    return order


@dataclass(frozen=True)
class RowSplit:
    """How a node's rows are cut: `chunks` tiles of `in_rows` input rows,
    each writing `out_rows` output rows (collectives scale the output)."""
    chunks: int
    in_rows: int
    out_rows: int

    def tiles_covering(self, lo, hi):
        """Tiles whose output rows meet [lo, hi). A consumer range past the
        produced rows maps to the last tile (the conservative choice of the
        reference's geometry, fixed.py:121-124)."""
        first = lo // self.out_rows
        if first >= self.chunks:
            return [self.chunks - 1]
        last = min((hi - 1) // self.out_rows, self.chunks - 1)
        return list(range(first, last + 1))


def row_splits(dag, chunking, nranks):
    """RowSplit of every node, checking that the cuts are whole rows."""
    out = {}
    for n in dag.nodes:
        k = chunking.get(n.name, 1)
        rows, produced = node_rows(n), out_rows(n, nranks)
        if rows % k:
            raise ValueError("%s: node %s rows=%d not divisible by chunks=%d" % (dag.name, n.name, rows, k))
        if produced % k:
            raise ValueError("%s: node %s output rows %d not divisible by chunks=%d" % (dag.name, n.name, produced, k))
        if n.op == "reducescatter" and (rows // k) % nranks:
            raise ValueError("%s: reducescatter %s rows per chunk must divide by nranks=%d"
                             % (dag.name, n.name, nranks))
        out[n.name] = RowSplit(k, rows // k, produced // k)
    return out


def _task(node, tile, split):
    return {"node": node, "tile": tile, "wait": [], "publish": False, "in_row_off": tile * split.in_rows,
            "in_rows": split.in_rows, "out_row_off": tile * split.out_rows}


def build_fixed_schedule(dag, chunking=None, nranks=1, method="fixed"):
    """DAG + per-node chunk counts -> schedule.json content (dict), the
    format of the reference's fixed-plan writer
    (python/kernrelay/_vendor/scheduler/fixed.py:64-156).

    Each node's rows are cut into equal tiles. A consumer tile waits on every
    producer tile whose output rows meet its input rows, but only across
    streams (one stream's FIFO already orders its tasks), and those producer
    tiles publish. Tasks join their op's stream in dependency order."""
    chunking = {k: int(v) for k, v in dict(chunking or {}).items() if int(v) > 0}
    by_name = dag.node_map
    unknown = sorted(set(chunking) - set(by_name))
    if unknown:
        raise ValueError("%s: chunking names unknown nodes %s" % (dag.name, unknown))
    sinks_only = [e for e in dag.edges if by_name[e.src].op == "cast"]
    if sinks_only:
        raise ValueError("%s: a cast output may only be a sink, not consumed by %s" % (dag.name, sinks_only[0].dst))
    splits = row_splits(dag, chunking, nranks)
    tasks = {(n.name, t): _task(n.name, t, splits[n.name]) for n in dag.nodes for t in range(splits[n.name].chunks)}

    for e in dag.edges:
        src, dst = by_name[e.src], by_name[e.dst]
        if node_rows(dst) > out_rows(src, nranks):
            raise ValueError("%s: edge %s->%s consumer reads %d rows but the producer writes %d"
                             % (dag.name, e.src, e.dst, node_rows(dst), out_rows(src, nranks)))
        if stream_of(src.op) == stream_of(dst.op):
            continue
        ps, cs = splits[src.name], splits[dst.name]
        for j in range(cs.chunks):
            for k in ps.tiles_covering(j * cs.in_rows, (j + 1) * cs.in_rows):
                tasks[(dst.name, j)]["wait"].append([src.name, k])
                tasks[(src.name, k)]["publish"] = True

    streams = {}
    for name in topo_order(dag):
        lane = streams.setdefault(stream_of(by_name[name].op), [])
        lane.extend(tasks[(name, t)] for t in range(splits[name].chunks))

    nodes = []
    for n in dag.nodes:
        k = splits[n.name].chunks
        entry = {"id": n.name, "op": n.op, "engine": stream_of(n.op), "dtype": n.dtype, "tiles": k,
                 "split": k > 1, "preds": [e.src for e in dag.edges if e.dst == n.name], "iters": 1, "blocks": 1}
        entry.update(node_dims(n))
        entry.update(n.extra)
        nodes.append(entry)
    return {"dag": dag.name, "group": method, "nranks": int(nranks), "nodes": nodes,
            "streams": {k: v for k, v in streams.items() if v},
            "chunking": {k: v for k, v in chunking.items() if v > 1}, "fallback": ""}


# Which stream's head goes first when several could run next in the serial
# baseline (the reference's precedence, python/kernrelay/schedule.py:67-105):
# mixed work, then matrix, vector, CPU and collective streams; "compute" is
# another name of "aicore".
STREAM_PRECEDENCE = ("aicore", "aic", "aiv", "aicpu", "hccl")


def _precedence(stream):
    stream = "aicore" if stream == "compute" else stream
    return STREAM_PRECEDENCE.index(stream) if stream in STREAM_PRECEDENCE else len(STREAM_PRECEDENCE)


def serial_schedule(dag, nranks=1):
    """Serial baseline: every tile of the unsplit schedule on one ``aicore``
    stream, no waits or publishes. The per-stream FIFOs of the unsplit
    schedule are merged: a stream's head may go once every task it waits on
    has gone, and of the heads that may go, the stream of highest precedence
    goes first."""
    base = build_fixed_schedule(dag, {}, nranks=nranks, method="serial")
    lanes = sorted(base["streams"].items(), key=lambda kv: _precedence(kv[0]))
    heads = [0] * len(lanes)
    placed, merged = set(), []
    total = sum(len(seq) for _, seq in lanes)
    while len(merged) < total:
        for i, (_, seq) in enumerate(lanes):
            if heads[i] < len(seq) and all((w[0], int(w[1])) in placed for w in seq[heads[i]].get("wait") or []):
                t = seq[heads[i]]
                heads[i] += 1
                placed.add((t["node"], int(t.get("tile", 0))))
                merged.append(dict(t, wait=[], publish=False))
                break
        else:
            raise RuntimeError("%s: the serial baseline cannot order its streams (wait cycle)" % dag.name)
    out = dict(base)
    out.update(streams={"aicore": merged}, group="serial", chunking={})
    return out


def validate_schedule(sched):
    """Structural checks of a schedule.json dict (the executor stays the
    authority): node ids, stream names, tasks, waits on publishing tasks and
    a happens-before order without cycles (stream FIFO + waits). Returns the
    list of problems found."""
    errors = []
    ids = [n.get("id") for n in sched.get("nodes") or []]
    if len(ids) != len(set(ids)):
        errors.append("duplicate node ids")
    streams = sched.get("streams") or {}
    if not streams:
        errors.append("no streams")
    where, publishing = {}, set()
    before = {}  # task -> tasks that must finish first
    for engine, seq in streams.items():
        if engine not in ENGINES:
            errors.append("unknown stream %r" % engine)
        if not isinstance(seq, list):
            errors.append("stream %r is not a task list" % engine)
            continue
        prev = None
        for t in seq:
            key = (t.get("node"), int(t.get("tile", 0)))
            if key[0] not in ids:
                errors.append("stream %s task names unknown node %r" % (engine, key[0]))
            if key in where:
                errors.append("node %s tile %d repeated on streams %s/%s" % (key[0], key[1], where[key], engine))
            where[key] = engine
            if int(t.get("in_rows", 1)) <= 0:
                errors.append("node %s tile %d has in_rows <= 0" % key)
            if t.get("publish"):
                publishing.add(key)
            before.setdefault(key, set())
            if prev is not None:
                before[key].add(prev)
            prev = key
    for seq in streams.values():
        for t in seq if isinstance(seq, list) else []:
            key = (t.get("node"), int(t.get("tile", 0)))
            for w in t.get("wait") or []:
                dep = (w[0], int(w[1]))
                if dep not in where:
                    errors.append("node %s tile %d waits on missing task %s#%s" % (key[0], key[1], dep[0], dep[1]))
                    continue
                if dep not in publishing:
                    errors.append("node %s tile %d waits on %s#%s which never publishes"
                                  % (key[0], key[1], dep[0], dep[1]))
                before[key].add(dep)
    # a cycle in the happens-before relation: iterative three-colour DFS
    state = {}
    for root in before:
        if state.get(root):
            continue
        stack = [(root, iter(before[root]))]
        state[root] = 1
        while stack:
            node, deps = stack[-1]
            nxt = next(deps, None)
            if nxt is None:
                state[node] = 2
                stack.pop()
            elif state.get(nxt) == 1:
                errors.append("schedule has a wait cycle")
                return errors
            elif not state.get(nxt):
                state[nxt] = 1
                stack.append((nxt, iter(before.get(nxt, ()))))
    return errors


def invalid_variants(sched):
    """Broken copies of a valid schedule, each paired with the error marker
    the executor must reject it with (the four cases of the reference's E0
    rejection gate, python/kernrelay/schedule.py:185-222, whose markers are
    the executor's interface):
      duplicate_engine  a second name for the mixed stream holds tasks too
      ghost_task        a task of a node the schedule does not declare
      wait_cycle        the first tasks of two streams wait on each other
      row_overflow      a tile reads far past its node's rows"""
    out = {}
    named = [k for k, v in sched["streams"].items() if v]

    dup = copy.deepcopy(sched)
    moved = dup["streams"].pop(named[0])
    dup["streams"]["aicore"] = []
    dup["streams"]["compute"] = moved
    out["duplicate_engine"] = (dup, "duplicate engine stream")

    ghost = copy.deepcopy(sched)
    ghost["streams"][named[0]].append(
        {"node": "__ghost__", "tile": 0, "wait": [], "publish": False, "in_row_off": 0, "in_rows": 1})
    out["ghost_task"] = (ghost, "missing plan for task")

    if len(named) >= 2:
        cyc = copy.deepcopy(sched)
        a, b = cyc["streams"][named[0]][0], cyc["streams"][named[1]][0]
        for x, y in ((a, b), (b, a)):
            x["publish"] = True
            x.setdefault("wait", []).append([y["node"], int(y.get("tile", 0))])
        out["wait_cycle"] = (cyc, "wait cycle")

        over = copy.deepcopy(sched)
        later = [t for seq in over["streams"].values() for t in seq if t.get("in_row_off", 0) > 0]
        if later:
            later[0]["in_rows"] = int(later[0]["in_rows"]) + 10 ** 9
            out["row_overflow"] = (over, "exceed")
    return out


def dump_schedule(sched, path):
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(sched, indent=1), encoding="utf-8")
    return path
