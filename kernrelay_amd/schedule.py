"""DAG model and fixed row-split schedules consumed by kr_plan_run.

The schedule.json format, the tile geometry and the rejection markers are
the reference's interface for this path; the code is this module's own:

* ``build_fixed_schedule`` — the schedule the reference's fixed-plan writer
  emits (python/kernrelay/_vendor/scheduler/fixed.py:64-156), built as a
  relation: every node's input rows cut evenly into its chunk count; a
  consumer tile waits on the producer tiles whose output rows meet its
  input rows (the last producer tile when none do), across streams only; a
  task publishes exactly when something waits on it; each stream's FIFO is
  its tasks sorted by (topological rank of the node, tile), declaration
  order breaking ties between nodes;
* ``serial_schedule`` — the reference's serial baseline
  (python/kernrelay/schedule.py:67-105) as a list schedule over the unsplit
  schedule's happens-before graph, ties going to the stream of higher
  precedence, then to the earlier FIFO position;
* ``validate_schedule`` / ``invalid_variants`` — structural checks that name
  the offending task or cycle, and broken schedules for the four executor
  error markers the reference's E0 gate expects
  (python/kernrelay/schedule.py:108-222).

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


TaskKey = tuple  # (node name, tile index)


def _key(task):
    """(node, tile) of a schedule.json task record."""
    return task.get("node"), int(task.get("tile", 0))


def _cross_stream_waits(dag, splits):
    """The wait relation of a row-tiled DAG: {consumer task: [producer
    tasks]}. Only edges whose two ends run on different streams wait (a
    stream's FIFO already orders the rest). A consumer tile waits on the
    producer tiles whose output rows meet its input rows, taken edge by
    edge in the DAG's edge order, tiles ascending."""
    by_name = dag.node_map
    relation = {}
    for e in dag.edges:
        if stream_of(by_name[e.src].op) == stream_of(by_name[e.dst].op):
            continue
        made, used = splits[e.src], splits[e.dst]
        for j in range(used.chunks):
            lo = j * used.in_rows
            relation.setdefault((e.dst, j), []).extend(
                (e.src, k) for k in made.tiles_covering(lo, lo + used.in_rows))
    return relation


def _node_entry(node, chunks, preds):
    """schedule.json "nodes" record: the executor's fields for one node."""
    entry = dict(id=node.name, op=node.op, engine=stream_of(node.op), dtype=node.dtype, tiles=chunks,
                 split=chunks > 1, preds=preds, iters=1, blocks=1)
    entry.update(node_dims(node))
    entry.update(node.extra)
    return entry


def build_fixed_schedule(dag, chunking=None, nranks=1, method="fixed"):
    """DAG + per-node chunk counts -> schedule.json content (dict), in the
    format the reference's fixed-plan writer emits
    (python/kernrelay/_vendor/scheduler/fixed.py:64-156).

    Built as a relation rather than task by task: every (node, tile) task
    gets its equal share of the node's rows; the wait relation comes from
    the row cuts (`_cross_stream_waits`); a task publishes exactly when some
    task waits on it; and each stream's FIFO is the set of its tasks sorted
    by (topological rank of the node, tile)."""
    chunking = {k: int(v) for k, v in dict(chunking or {}).items() if int(v) > 0}
    by_name = dag.node_map
    unknown = sorted(set(chunking) - set(by_name))
    if unknown:
        raise ValueError("%s: chunking names unknown nodes %s" % (dag.name, unknown))
    for e in dag.edges:
        src, dst = by_name[e.src], by_name[e.dst]
        if src.op == "cast":
            raise ValueError("%s: a cast output may only be a sink, not consumed by %s" % (dag.name, e.dst))
        if node_rows(dst) > out_rows(src, nranks):
            raise ValueError("%s: edge %s->%s consumer reads %d rows but the producer writes %d"
                             % (dag.name, e.src, e.dst, node_rows(dst), out_rows(src, nranks)))
    splits = row_splits(dag, chunking, nranks)
    waits = _cross_stream_waits(dag, splits)
    waited_on = {w for ws in waits.values() for w in ws}
    rank = {name: r for r, name in enumerate(topo_order(dag))}
    keys = sorted(((n.name, t) for n in dag.nodes for t in range(splits[n.name].chunks)),
                  key=lambda k: (rank[k[0]], k[1]))
    streams = {}
    for name, tile in keys:
        cut = splits[name]
        streams.setdefault(stream_of(by_name[name].op), []).append({
            "node": name, "tile": tile, "wait": [list(w) for w in waits.get((name, tile), [])],
            "publish": (name, tile) in waited_on, "in_row_off": tile * cut.in_rows, "in_rows": cut.in_rows,
            "out_row_off": tile * cut.out_rows})
    preds = {n.name: [] for n in dag.nodes}
    for e in dag.edges:
        preds[e.dst].append(e.src)
    return {"dag": dag.name, "group": method, "nranks": int(nranks),
            "nodes": [_node_entry(n, splits[n.name].chunks, preds[n.name]) for n in dag.nodes],
            "streams": streams, "chunking": {k: v for k, v in chunking.items() if v > 1}, "fallback": ""}


def _stream_precedence(stream):
    """Serial tie-break between streams: the order of ENGINES (mixed work,
    matrix, vector, CPU, collectives); "compute" is the mixed stream's other
    name, unknown names go last."""
    stream = "aicore" if stream == "compute" else stream
    return ENGINES.index(stream) if stream in ENGINES else len(ENGINES)


def _happens_before(streams):
    """{task: set of tasks that must finish first} of a schedule's streams:
    each task's FIFO predecessor and the tasks it waits on."""
    before = {}
    for seq in streams.values():
        prev = None
        for t in seq:
            deps = before.setdefault(_key(t), set())
            deps.update((w[0], int(w[1])) for w in t.get("wait") or [])
            if prev is not None:
                deps.add(prev)
            prev = _key(t)
    return before


def serial_schedule(dag, nranks=1):
    """Serial baseline (the reference's, python/kernrelay/schedule.py:67-105):
    every task of the unsplit schedule on one ``aicore`` stream, no waits or
    publishes. The order is a list schedule of the unsplit schedule's
    happens-before graph: of the tasks whose predecessors have all gone, the
    one with the smallest (stream precedence, FIFO position) goes next."""
    import heapq
    base = build_fixed_schedule(dag, {}, nranks=nranks, method="serial")
    record, priority = {}, {}
    for stream, seq in base["streams"].items():
        for pos, t in enumerate(seq):
            record[_key(t)] = t
            priority[_key(t)] = (_stream_precedence(stream), pos)
    before = _happens_before(base["streams"])
    pending = {k: len(v) for k, v in before.items()}
    after = {k: [] for k in before}
    for k, deps in before.items():
        for d in deps:
            after[d].append(k)
    ready = [(priority[k], k) for k, n in pending.items() if n == 0]
    heapq.heapify(ready)
    order = []
    while ready:
        _, k = heapq.heappop(ready)
        order.append(dict(record[k], wait=[], publish=False))
        for nxt in after[k]:
            pending[nxt] -= 1
            if pending[nxt] == 0:
                heapq.heappush(ready, (priority[nxt], nxt))
    if len(order) != len(record):
        raise RuntimeError("%s: the serial baseline cannot order its streams (wait cycle)" % dag.name)
    out = dict(base)
    out.update(streams={"aicore": order}, group="serial", chunking={})
    return out


def _find_cycle(before):
    """One cycle of a {task: predecessors} graph as a task list (first ==
    last), or None. Depth-first, iterative, with the path kept on a stack."""
    colour = {}
    for root in before:
        if root in colour:
            continue
        path, iters = [root], [iter(sorted(before[root], key=repr))]
        colour[root] = "open"
        while path:
            nxt = next(iters[-1], None)
            if nxt is None:
                colour[path.pop()] = "done"
                iters.pop()
            elif colour.get(nxt) == "open":
                return path[path.index(nxt):] + [nxt]
            elif nxt not in colour:
                colour[nxt] = "open"
                path.append(nxt)
                iters.append(iter(sorted(before.get(nxt, ()), key=repr)))
    return None


def validate_schedule(sched):
    """Problems found in a schedule.json dict, as messages (empty: none);
    the executor stays the authority. Checked: node ids unique; streams
    named for engines and holding task lists; every task of a declared
    node, on one stream only, with in_rows > 0; every wait on an existing
    task that publishes; and the happens-before graph (FIFO + waits) free of
    cycles, one of which is named when present."""
    problems = []
    declared = [n.get("id") for n in sched.get("nodes") or []]
    if len(declared) != len(set(declared)):
        problems.append("node ids are not unique")
    streams = sched.get("streams") or {}
    if not streams:
        problems.append("the schedule has no streams")
    lists = {}
    for name, seq in streams.items():
        if name not in ENGINES:
            problems.append("stream %r is not an engine" % name)
        if isinstance(seq, list):
            lists[name] = seq
        else:
            problems.append("stream %r is not a task list" % name)
    home = {}
    for name, seq in lists.items():
        for t in seq:
            k = _key(t)
            if k[0] not in declared:
                problems.append("a task on stream %s belongs to unknown node %r" % (name, k[0]))
            if k in home:
                problems.append("task %s#%d repeated on streams %s and %s" % (k[0], k[1], home[k], name))
            home.setdefault(k, name)
            if int(t.get("in_rows", 1)) <= 0:
                problems.append("task %s#%d reads no rows" % k)
    publishes = {_key(t) for seq in lists.values() for t in seq if t.get("publish")}
    for seq in lists.values():
        for t in seq:
            for w in t.get("wait") or []:
                dep = (w[0], int(w[1]))
                if dep not in home:
                    problems.append("task %s#%d waits on %s#%d, which no stream runs" % (_key(t) + dep))
                elif dep not in publishes:
                    problems.append("task %s#%d waits on %s#%d, which never publishes" % (_key(t) + dep))
    cycle = _find_cycle({k: {d for d in v if d in home} for k, v in _happens_before(lists).items()})
    if cycle:
        problems.append("wait cycle: " + " -> ".join("%s#%d" % k for k in cycle))
    return problems


def _task_streams(sched):
    return [name for name, seq in sched["streams"].items() if seq]


def _alias_mixed_stream(sched):
    """The mixed stream under both of its names (an empty ``aicore`` and an
    empty ``compute`` lane beside the others)."""
    sched["streams"].setdefault("aicore", [])
    sched["streams"]["compute"] = []
    return sched


def _undeclared_node(sched):
    """A copy of the last task of the first stream, for a node the schedule
    does not declare."""
    seq = sched["streams"][_task_streams(sched)[0]]
    seq.append(dict(seq[-1], node="undeclared_node", wait=[], publish=False))
    return sched


def _crossed_waits(sched):
    """The first task of the second stream waits on the last task of the
    first stream, which waits on it in turn."""
    first, second = (sched["streams"][s] for s in _task_streams(sched)[:2])
    tail, head = first[-1], second[0]
    for x, y in ((tail, head), (head, tail)):
        x["publish"] = True
        x["wait"] = list(x.get("wait") or []) + [list(_key(y))]
    return sched


def _shifted_past_rows(sched):
    """The last task of the first stream reads starting past every row that
    any node of the schedule produces."""
    past = sum(int(n["rows"]) for n in sched["nodes"]) * max(1, int(sched.get("nranks", 1))) + 1
    sched["streams"][_task_streams(sched)[0]][-1]["in_row_off"] = past
    return sched


# The reference's four executor rejection cases
# (python/kernrelay/schedule.py:185-222): label -> (mutation, the marker the
# executor's error must contain, streams with tasks the mutation needs).
# The markers are the executor's interface; the mutations are this module's.
REJECTION_CASES = {
    "duplicate_engine": (_alias_mixed_stream, "duplicate engine stream", 1),
    "ghost_task": (_undeclared_node, "missing plan for task", 1),
    "wait_cycle": (_crossed_waits, "wait cycle", 2),
    "row_overflow": (_shifted_past_rows, "exceed", 1),
}


def invalid_variants(sched):
    """Broken copies of a valid schedule: {label: (schedule, marker)}, the
    executor must reject each with an error containing its marker. A case
    that needs more task-holding streams than the schedule has is left
    out."""
    have = len(_task_streams(sched))
    return {label: (mutate(copy.deepcopy(sched)), marker)
            for label, (mutate, marker, needs) in REJECTION_CASES.items() if have >= needs}


def dump_schedule(sched, path):
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(sched, indent=1), encoding="utf-8")
    return path
