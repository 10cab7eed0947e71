"""The schedule writer (kernrelay_amd/schedule.py) on the CPU: row geometry
against brute-force interval intersection, the serial baseline as a
topological order on one stream, and the structural validator against
schedules broken on purpose."""

import random

import pytest

from kernrelay_amd import schedule, workloads


def brute_tiles(chunks, out_rows, lo, hi):
    hits = [k for k in range(chunks) if max(lo, k * out_rows) < min(hi, (k + 1) * out_rows)]
    return hits or [chunks - 1]


def test_tiles_covering_matches_brute_force():
    rnd = random.Random(3)
    for _ in range(5000):
        chunks = rnd.choice([1, 2, 3, 4, 8])
        out_rows = rnd.choice([1, 8, 64, 100])
        lo = rnd.randrange(0, chunks * out_rows + 50)
        hi = lo + rnd.randrange(1, 300)
        got = schedule.RowSplit(chunks, out_rows, out_rows).tiles_covering(lo, hi)
        assert got == brute_tiles(chunks, out_rows, lo, hi), (chunks, out_rows, lo, hi)


def mm_chain(M=1024):
    return schedule.dag_from_dict(workloads.mm_consumers_dag("mn", M, 256, 256, ["gelu", "softmax"]))


@pytest.mark.parametrize("chunking", [{"mm": 8, "gelu": 4, "softmax": 2}, {"mm": 2, "gelu": 8, "softmax": 8},
                                      {"mm": 4, "gelu": 1}, {}])
def test_fixed_schedule_row_geometry(chunking):
    dag = mm_chain()
    sched = schedule.build_fixed_schedule(dag, chunking)
    assert schedule.validate_schedule(sched) == []
    tasks = {(t["node"], t["tile"]): t for seq in sched["streams"].values() for t in seq}
    k_mm = chunking.get("mm", 1)
    per_mm = 1024 // k_mm
    waited = set()
    for name in ("gelu", "softmax"):
        k = chunking.get(name, 1)
        per = 1024 // k
        for j in range(k):
            t = tasks[(name, j)]
            assert (t["in_row_off"], t["in_rows"]) == (j * per, per)
            want = brute_tiles(k_mm, per_mm, j * per, (j + 1) * per)
            assert sorted(w[1] for w in t["wait"]) == want and all(w[0] == "mm" for w in t["wait"])
            waited |= {("mm", w) for w in want}
    # a producer tile publishes exactly when some consumer tile waits on it
    assert {k for k, t in tasks.items() if t["publish"]} == waited
    # streams: matrix work on aic, vector work on aiv, tiles in order
    assert [t["node"] for t in sched["streams"]["aic"]] == ["mm"] * k_mm
    assert [t["tile"] for t in sched["streams"]["aic"]] == list(range(k_mm))


def test_same_stream_edges_carry_no_waits():
    raw = {"name": "vv", "nodes": [{"name": "a", "op": "gelu", "shape": {"rows": 512, "cols": 64}},
                                   {"name": "b", "op": "softmax", "shape": {"rows": 512, "cols": 64}}],
           "edges": [{"src": "a", "dst": "b"}]}
    sched = schedule.build_fixed_schedule(schedule.dag_from_dict(raw), {"a": 4, "b": 2})
    assert all(not t["wait"] and not t["publish"] for t in sched["streams"]["aiv"])
    assert [(t["node"], t["tile"]) for t in sched["streams"]["aiv"]] == [("a", i) for i in range(4)] + \
        [("b", 0), ("b", 1)]


def test_serial_schedule_is_one_topological_stream():
    rnd = random.Random(5)
    for trial in range(200):
        n = rnd.randint(1, 7)
        nodes = [{"name": "n0", "op": "matmul", "shape": {"M": 256, "K": 64, "N": 64}}]
        edges = []
        for j in range(1, n):
            op = rnd.choice(["matmul", "gelu", "softmax", "add"])
            shape = {"M": 256, "K": 64, "N": 64} if op == "matmul" else {"rows": 256, "cols": 64}
            nodes.append({"name": "n%d" % j, "op": op, "shape": shape})
            for p in rnd.sample(range(j), rnd.randint(1, min(2, j))):
                edges.append({"src": "n%d" % p, "dst": "n%d" % j})
        dag = schedule.dag_from_dict({"name": "t%d" % trial, "nodes": nodes, "edges": edges})
        s = schedule.serial_schedule(dag)
        assert list(s["streams"]) == ["aicore"] and s["group"] == "serial"
        seq = [t["node"] for t in s["streams"]["aicore"]]
        assert sorted(seq) == sorted(nd["name"] for nd in nodes)
        pos = {name: i for i, name in enumerate(seq)}
        assert all(pos[e["src"]] < pos[e["dst"]] for e in edges)
        assert all(not t["wait"] and not t["publish"] for t in s["streams"]["aicore"])


def test_topo_order_prefers_declaration_order():
    raw = {"name": "o", "nodes": [{"name": x, "op": "gelu", "shape": {"rows": 8, "cols": 8}} for x in "dcba"],
           "edges": [{"src": "c", "dst": "a"}]}
    assert schedule.topo_order(schedule.dag_from_dict(raw)) == ["d", "c", "b", "a"]
    nodes = schedule.dag_from_dict(raw).nodes
    with pytest.raises(ValueError, match="cycle"):
        schedule.topo_order(schedule.Dag("o", "", nodes, [schedule.Edge("c", "a"), schedule.Edge("a", "c")]))


def test_validator_flags_broken_schedules(tmp_path):
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, {"mm": 2, "gelu": 2})
    assert schedule.validate_schedule(sched) == []
    bad = schedule.invalid_variants(sched)
    assert set(bad) == {"duplicate_engine", "ghost_task", "wait_cycle", "row_overflow"}
    assert any("wait cycle" in e for e in schedule.validate_schedule(bad["wait_cycle"][0]))
    assert any("unknown node" in e for e in schedule.validate_schedule(bad["ghost_task"][0]))
    # a wait on a task that never publishes
    import copy
    quiet = copy.deepcopy(sched)
    for t in quiet["streams"]["aic"]:
        t["publish"] = False
    assert any("never publishes" in e for e in schedule.validate_schedule(quiet))
    # the same task on two streams
    twice = copy.deepcopy(sched)
    twice["streams"]["aiv"].append(dict(twice["streams"]["aic"][0]))
    assert any("repeated" in e for e in schedule.validate_schedule(twice))


def test_rows_must_divide():
    with pytest.raises(ValueError, match="not divisible"):
        schedule.build_fixed_schedule(mm_chain(1000), {"mm": 3})


def test_validator_names_the_cycle_and_every_case_trips_it(tmp_path):
    """The cycle message lists the tasks on it; each broken variant is flagged
    by the validator too (the executor's markers are checked in test_abi)."""
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, {"mm": 2, "gelu": 2})
    bad = schedule.invalid_variants(sched)
    msg = [e for e in schedule.validate_schedule(bad["wait_cycle"][0]) if "wait cycle" in e]
    assert len(msg) == 1
    path = msg[0].split(": ", 1)[1].split(" -> ")
    assert path[0] == path[-1] and len(path) >= 3
    assert set(path) >= {"mm#1", "gelu#0"}
    assert any("not an engine" in e for e in schedule.validate_schedule(bad["duplicate_engine"][0]))
    assert schedule.validate_schedule(bad["row_overflow"][0]) == []  # rows are the executor's check


def test_single_stream_schedule_variants():
    """A schedule with one task-holding stream (the serial baseline) still
    yields the cases that need one stream; the wait cycle needs two."""
    sched = schedule.serial_schedule(mm_chain(512))
    bad = schedule.invalid_variants(sched)
    assert set(bad) == {"duplicate_engine", "ghost_task", "row_overflow"}
    over = bad["row_overflow"][0]["streams"]["aicore"][-1]
    assert over["in_row_off"] > max(n["rows"] for n in sched["nodes"])


def test_serial_schedule_is_a_priority_list_schedule():
    """On random DAGs the serial order respects every happens-before edge of
    the unsplit schedule, and whenever a task goes, no ready task of a
    stream with higher precedence (or earlier in the same FIFO) was left."""
    import random
    rng = random.Random(3)
    ops = ["matmul", "gelu", "softmax", "cast", "add", "topk", "allreduce"]
    for trial in range(150):
        n = rng.randint(1, 6)
        nodes = []
        for i in range(n):
            op = rng.choice(ops)
            shape = {"M": 128, "K": 64, "N": 64} if op == "matmul" else (
                {"rows": 128, "cols": 64, "k": 2} if op == "topk" else {"rows": 128, "cols": 64})
            nodes.append({"name": "n%d" % i, "op": op, "shape": shape})
        edges = [{"src": "n%d" % i, "dst": "n%d" % j} for i in range(n) for j in range(i + 1, n)
                 if rng.random() < 0.4 and nodes[i]["op"] != "cast"]
        dag = schedule.dag_from_dict({"name": "t%d" % trial, "nodes": nodes, "edges": edges})
        base = schedule.build_fixed_schedule(dag, {})
        prio = {}
        before = {}
        for st, seq in base["streams"].items():
            for pos, t in enumerate(seq):
                k = (t["node"], t["tile"])
                prio[k] = (schedule.ENGINES.index(st), pos)
                before[k] = {tuple(w) for w in t["wait"]} | ({(seq[pos - 1]["node"], seq[pos - 1]["tile"])} if pos else set())
        order = [(t["node"], t["tile"]) for t in schedule.serial_schedule(dag)["streams"]["aicore"]]
        assert sorted(order) == sorted(prio)
        done = set()
        for k in order:
            assert before[k] <= done
            ready = [r for r in prio if r not in done and before[r] <= done]
            assert prio[k] == min(prio[r] for r in ready)
            done.add(k)
