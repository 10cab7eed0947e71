"""kr_plan_run end to end on the GPU: DAG schedules (serial, B0, split at k)
through the C ABI, checked against the oracle, against each other (bit-exact)
and against the reference's recorded checksums."""

import os

import numpy as np
import pytest
import torch

from kernrelay_amd import libapi, schedule, workloads
from oracle import dag_eval
from tests.conftest import announce
from tests.test_oracle_dag import E9_KATS, KATS, kat_dag, ln_mm_dag, ref_dag

pytestmark = pytest.mark.gpu


def run(sched, tmp, name, mode="direct", env=None, iters=2, warmup=1):
    """Run a schedule; returns (result, {node: raw 16-bit words})."""
    path = schedule.dump_schedule(sched, tmp / (name + ".json"))
    dump = tmp / ("dump_" + name)
    dump.mkdir(exist_ok=True)
    saved = {}
    env = dict(env or {})
    env["KR_DUMP_DIR"] = str(dump)
    for k, v in env.items():
        saved[k] = os.environ.get(k)
        os.environ[k] = v
    try:
        announce("plan_run %s mode=%s env=%s" % (name, mode, {k: v for k, v in env.items() if k != "KR_DUMP_DIR"}))
        r = libapi.plan_run(path, devices="0", mode=mode, iters=iters, warmup=warmup,
                            out_json=tmp / (name + "_out.json"))
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    assert r["_rc"] == 0, r
    outs = {n["id"]: np.fromfile(dump / (n["id"] + ".bin"), dtype=np.uint16) for n in sched["nodes"]}
    return r, outs


def as_float(words, node):
    odt = dag_eval.out_dtype(node)
    if odt == "fp32":
        return words.view(np.float32).astype(np.float64)
    if odt == "bf16":
        return torch.from_numpy(words.view(np.int16).copy()).view(torch.bfloat16).double().numpy()
    return words.view(np.float16).astype(np.float64)


def assert_close_to_oracle(sched, outs, rows=None):
    ref = dag_eval.node_outputs(sched, rows=rows)
    for n in sched["nodes"]:
        r = ref[n["id"]].double().numpy().reshape(-1)
        g = as_float(outs[n["id"]], n)[: r.size]
        err = np.abs(g - r)
        bound = 2e-2 + 1e-2 * np.abs(r)
        assert np.all(err <= bound), (n["id"], float(err.max()))


def test_tiny_mm_gelu_relay(gpu, tmp_path):
    dag = workloads.tiny_mm_gelu(tmp_path)
    v = workloads.variants(dag, 2)
    base = None
    for name, sched in v.items():
        for mode in ("direct", "graph_per_stream"):
            r, outs = run(sched, tmp_path, "%s_%s" % (name, mode), mode=mode)
            assert r["ok"] and r["gate_timeouts"] == 0
            if base is None:
                base = outs
                assert_close_to_oracle(sched, outs)
            for k in outs:
                assert np.array_equal(outs[k], base[k]), (name, mode, k)


def test_event_sync_matches_flags(gpu, tmp_path):
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, {"mm": 2, "gelu": 2})
    _, flag = run(sched, tmp_path, "flag")
    for mode in ("direct", "graph"):
        _, ev = run(sched, tmp_path, "event_" + mode, mode=mode, env={"KR_SYNC": "event"})
        for k in flag:
            assert np.array_equal(flag[k], ev[k])


@pytest.mark.parametrize("chunking", [{"mm": 2, "gelu": 2}, {"mm": 4, "gelu": 2}, {"mm": 1, "gelu": 4}])
def test_graph_segment_matches_flags(gpu, tmp_path, chunking):
    """graph_segment (the reference's NHP_GRAPH_SEGMENT): each stream's tasks
    cut into graphs at every cross-stream wait and after every publish, joined
    by events; the outputs equal the flag relay's bit for bit, repeated runs
    included."""
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, chunking)
    _, flag = run(sched, tmp_path, "flag")
    r, seg = run(sched, tmp_path, "segment", mode="graph_segment", iters=3, warmup=1)
    assert r["ok"] and r["sync"] == "event" and r["mode"] == "graph_segment"
    for k in flag:
        assert np.array_equal(flag[k], seg[k]), k


@pytest.mark.parametrize("name,consumers,expected", KATS[:2])
def test_graph_segment_reference_checksums(gpu, tmp_path, name, consumers, expected):
    """The reference's KAT DAGs (2 ranks, split at k=4) in graph_segment mode
    reproduce its recorded checksums."""
    dag = kat_dag(name, consumers)
    sched = schedule.build_fixed_schedule(dag, {n.name: 4 for n in dag.nodes}, nranks=2)
    path = schedule.dump_schedule(sched, tmp_path / "kat_seg.json")
    announce("plan_run KAT graph_segment " + name)
    r = libapi.plan_run(path, devices="0,0", mode="graph_segment", iters=2, warmup=1,
                        out_json=tmp_path / "kat_seg_out.json")
    assert r["_rc"] == 0 and r["ok"], r
    assert abs(r["checksum"] - expected) / abs(expected) < 1e-3, (r["checksum"], expected)


@pytest.mark.parametrize("name,consumers,k", [("f01_mm_gelu_c2", ["gelu"], 4), ("e3_mm_cast", ["cast"], 2),
                                              ("e3_mm_silu", ["silu"], 8)])
def test_epilogue_relay_bit_exact(gpu, tmp_path, name, consumers, k):
    """The in-register relay (KR_PLAN_EPILOGUE=1): the reference's e34 DAG
    split at k with its GELU / cast (fp16 -> fp32) / SiLU consumer computed
    in the GEMM's epilogue equals the serial schedule bit for bit (both
    outputs), runs no consumer launch and no relay edge, and reproduces the
    reference's checksum where it has one."""
    dag = workloads.e34_dag(name, consumers)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial", iters=1, warmup=0)
    sched = workloads.variants(dag, k)["split"]
    r, outs = run(sched, tmp_path, "epi", mode="graph_per_stream", env={"KR_PLAN_EPILOGUE": "1"})
    assert r["ok"] and r["epilogue_consumers"] == 1 and r["flag_edges"] == 0, r
    for node in base:
        assert np.array_equal(base[node], outs[node]), node
    expected = {kk[0]: kk[2] for kk in KATS}.get(name)
    if expected is not None:
        r2 = libapi.plan_run(schedule.dump_schedule(schedule.build_fixed_schedule(dag, {n.name: 4 for n in dag.nodes},
                                                                                  nranks=2), tmp_path / "kat.json"),
                             devices="0,0", mode="direct", iters=1, warmup=0, out_json=tmp_path / "kat_out.json")
        assert r2["_rc"] == 0 and r2["ok"]
        # (KR_PLAN_EPILOGUE is unset here: the plain relay's checksum)
        assert abs(r2["checksum"] - expected) / abs(expected) < 1e-3
        os.environ["KR_PLAN_EPILOGUE"] = "1"
        try:
            r3 = libapi.plan_run(tmp_path / "kat.json", devices="0,0", mode="direct", iters=1, warmup=0,
                                 out_json=tmp_path / "kat_out3.json")
        finally:
            del os.environ["KR_PLAN_EPILOGUE"]
        assert r3["_rc"] == 0 and r3["ok"] and r3["epilogue_consumers"] >= 1
        assert abs(r3["checksum"] - expected) / abs(expected) < 1e-3, (r3["checksum"], expected)


def test_wait_kernel_variant_matches(gpu, tmp_path):
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, {"mm": 2, "gelu": 2})
    _, fused = run(sched, tmp_path, "fused")
    _, kern = run(sched, tmp_path, "kern", env={"KR_RELAY_WAIT": "kernel"})
    for k in fused:
        assert np.array_equal(fused[k], kern[k])


@pytest.mark.parametrize("chunking", [{"mm": 8, "gelu": 4}, {"mm": 2, "gelu": 8}, {"mm": 4, "gelu": 1}])
def test_mn_row_geometry(gpu, tmp_path, chunking):
    dag = workloads.tiny_mm_gelu(tmp_path)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial")
    r, outs = run(schedule.build_fixed_schedule(dag, chunking), tmp_path, "mn")
    assert r["ok"]
    for k in base:
        assert np.array_equal(base[k], outs[k]), (chunking, k)


@pytest.mark.parametrize("name,consumers,expected", KATS)
def test_reference_checksums_on_gpu(gpu, tmp_path, name, consumers, expected):
    """The reference's own E3/E4 DAGs (fp16, 2 ranks, DetValue inputs) split at
    k=4 reproduce its recorded checksums within its consistency gate: mm ->
    gelu / softmax / both / cast, and the reverse edge LayerNorm -> mm."""
    dag = kat_dag(name, consumers)
    sched = schedule.build_fixed_schedule(dag, {n.name: 4 for n in dag.nodes}, nranks=2)
    path = schedule.dump_schedule(sched, tmp_path / "kat.json")
    announce("plan_run KAT " + name)
    r = libapi.plan_run(path, devices="0,0", mode="direct", iters=1, warmup=0, out_json=tmp_path / "kat_out.json")
    assert r["_rc"] == 0 and r["ok"], r
    assert abs(r["checksum"] - expected) / abs(expected) < 1e-3, (r["checksum"], expected)
    assert abs(r["checksum"] - dag_eval.checksum(sched)) / abs(expected) < 1e-3


@pytest.mark.parametrize("k", [4, 8])
@pytest.mark.parametrize("name,expected,tol", E9_KATS)
def test_e9_reference_checksums_on_gpu(gpu, tmp_path, name, expected, tol, k):
    """The reference's two-wave DAGs at its shapes (fp16 GEMMs over 32768
    rows, 2 ranks, DetValue inputs) split at k reproduce its recorded
    checksums (results/final/e9_raw.json) within its consistency gate, and
    the oracle's: two independent mm -> GELU chains, and mm -> GELU -> mm ->
    GELU, whose second GEMM waits on the GELU's published row tiles."""
    dag = workloads.e9_dag(name)
    sched = schedule.build_fixed_schedule(dag, {n.name: k for n in dag.nodes}, nranks=2)
    path = schedule.dump_schedule(sched, tmp_path / "e9.json")
    announce("plan_run E9 %s k=%d" % (name, k))
    r = libapi.plan_run(path, devices="0,0", mode="direct", iters=1, warmup=0, out_json=tmp_path / "e9_out.json")
    assert r["_rc"] == 0 and r["ok"] and r["gate_timeouts"] == 0, r
    ref = dag_eval.checksum(sched)
    announce("checksum %.7f, recorded %.7f, oracle %.7f" % (r["checksum"], expected, ref))
    assert abs(r["checksum"] - expected) / abs(expected) < 1e-3, (r["checksum"], expected)
    assert abs(r["checksum"] - ref) / abs(expected) < 1e-3, (r["checksum"], ref)


@pytest.mark.parametrize("name", ["e9_two_waves", "e9_chain2"])
def test_e9_variants_bit_exact(gpu, tmp_path, name):
    """The two-wave DAGs at 4096 rows: B0 and the relay split at k = 4 and 8
    (graph per stream, device flags), and the k = 4 split in the other
    executor modes (direct launches with flags or events, graph_segment),
    store every node's output bit for bit as the serial program does; the
    first 256 rows of every node against the oracle."""
    dag = workloads.e9_dag(name, M=4096)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial", iters=1, warmup=0)
    cases = [("b0", 1, "graph_per_stream", None), ("split", 4, "graph_per_stream", None),
             ("split", 8, "graph_per_stream", None), ("split", 4, "direct", None),
             ("split", 4, "direct", {"KR_SYNC": "event"}), ("split", 4, "graph_segment", None)]
    for vn, k, mode, env in cases:
        tag = "%s%d_%s%s" % (vn, k, mode, "_event" if env else "")
        r, outs = run(workloads.variants(dag, k)[vn], tmp_path, tag, mode=mode, env=env)
        assert r["ok"] and r["gate_timeouts"] == 0, (tag, r)
        if vn == "split" and r["sync"] == "flag":
            assert r["flag_edges"] > 0
        for node in base:
            assert np.array_equal(base[node], outs[node]), (tag, node)
    assert_close_to_oracle(schedule.serial_schedule(dag), base, rows=256)


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_fanout_4096_split_bit_exact(gpu, tmp_path, k):
    """mm -> {softmax, gelu, cast} at 4096^3 bf16: every split equals serial."""
    dag = workloads.mm_fanout(tmp_path)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial", iters=1, warmup=0)
    r, outs = run(workloads.variants(dag, k)["split"], tmp_path, "split%d" % k, mode="graph_per_stream")
    assert r["ok"] and r["gate_timeouts"] == 0
    for node in base:
        assert np.array_equal(base[node], outs[node]), (k, node)
    if k == 4:
        assert_close_to_oracle(schedule.serial_schedule(dag), outs, rows=256)


def test_qwen_consumers_as_dag(gpu, tmp_path):
    """The Qwen relay consumers (SwiGLU, Add+RMSNorm) behind a row-split GEMM."""
    inputs = workloads.write_inputs(tmp_path, 512, 256, 1024)
    raw = {"name": "mm_qwen_consumers", "nodes": [
        {"name": "mm", "op": "matmul", "shape": {"M": 512, "K": 256, "N": 1024}, "dtype": "bf16", "inputs": inputs},
        {"name": "swiglu", "op": "swiglu", "shape": {"rows": 512, "cols": 1024}, "dtype": "bf16"},
        {"name": "addnorm", "op": "add_rmsnorm", "shape": {"rows": 512, "cols": 1024}, "dtype": "bf16"}],
        "edges": [{"src": "mm", "dst": "swiglu"}, {"src": "mm", "dst": "addnorm"}]}
    dag = schedule.dag_from_dict(raw)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial")
    r, outs = run(schedule.build_fixed_schedule(dag, {"mm": 4, "swiglu": 4, "addnorm": 2}), tmp_path, "split")
    assert r["ok"]
    for k in base:
        assert np.array_equal(base[k], outs[k]), k
    assert_close_to_oracle(schedule.serial_schedule(dag), outs)


@pytest.mark.parametrize("k", [1, 4])
def test_fanout_b0_and_uncoalesced_match_serial(gpu, tmp_path, k):
    """B0 (two streams, unsplit) and the split run one launch per task
    (KR_PLAN_COALESCE=0, the reference's task granularity) give the serial
    bits, as the coalesced relay launches do."""
    dag = workloads.mm_fanout(tmp_path, M=1024, K=512, N=2048)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial", iters=1, warmup=0)
    v = workloads.variants(dag, k)
    for name, sched, env in (("b0", v["b0"], None), ("split_nc", v["split"], {"KR_PLAN_COALESCE": "0"}),
                             ("split_nofan", v["split"], {"KR_PLAN_FAN": "1"})):
        r, outs = run(sched, tmp_path, "%s%d" % (name, k), mode="graph_per_stream", env=env)
        assert r["ok"] and r["gate_timeouts"] == 0, (name, r)
        for node in base:
            assert np.array_equal(base[node], outs[node]), (name, k, node)


def test_fused_fanout_all_ops(gpu, tmp_path):
    """Four sibling consumers fused into one pass (rmsnorm, silu, cast to fp32,
    softmax) behind a GEMM released in 4 row tiles: each output equals its
    standalone kernel's bits and the oracle."""
    inputs = workloads.write_inputs(tmp_path, 512, 256, 1024)
    raw = workloads.mm_consumers_dag("fan4", 512, 256, 1024, ["rmsnorm", "silu", "cast", "softmax"],
                                     inputs=inputs, cast_to="fp32")
    dag = schedule.dag_from_dict(raw)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial")
    for k in (1, 2, 4):
        r, outs = run(workloads.variants(dag, k)["split"], tmp_path, "split%d" % k, mode="graph_per_stream")
        assert r["ok"] and r["gate_timeouts"] == 0 and r["flag_edges"] == 4 * k, r
        for node in base:
            assert np.array_equal(base[node], outs[node]), (k, node)
    assert_close_to_oracle(schedule.serial_schedule(dag), outs)


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_layernorm_to_gemm_relay(gpu, tmp_path, k):
    """The reverse edge (the reference's dags/e3_ln_mm.json at 4096 rows): a
    LayerNorm on the consumer stream releases k row tiles and the GEMM on the
    producer stream waits for the tiles of A each of its tiles reads. Split
    == serial bit for bit; both within the bf16 bar of the oracle."""
    raw = {"name": "ln_mm", "nodes": [
        {"name": "ln", "op": "layernorm", "engine": "aiv", "shape": {"rows": 4096, "cols": 2048}, "dtype": "bf16"},
        {"name": "mm", "op": "matmul", "engine": "aic", "shape": {"M": 4096, "K": 2048, "N": 2048}, "dtype": "bf16"}],
        "edges": [{"src": "ln", "dst": "mm", "kind": "data"}]}
    dag = schedule.dag_from_dict(raw)
    _, base = run(schedule.serial_schedule(dag), tmp_path, "serial")
    r, outs = run(schedule.build_fixed_schedule(dag, {"ln": k, "mm": k}), tmp_path, "split%d" % k,
                  mode="graph_per_stream")
    assert r["gate_timeouts"] == 0
    for name in ("ln", "mm"):
        assert np.array_equal(outs[name], base[name]), name
    assert_close_to_oracle(schedule.serial_schedule(dag), outs, rows=128)


@pytest.mark.parametrize("part", [1, 4])
def test_cu_partition_bit_exact(gpu, tmp_path, part):
    """KR_PLAN_PARTITION: lane 1 owns `part` CUs of every XCD and lane 0 the
    rest. The consumers wait for each producer tile in persistent grids on
    their own CUs, and a GEMM behind the other lane's producer waits in its
    own workgroups (the reverse edge, and the second GEMM of mm -> GELU ->
    mm -> GELU). Every node equals the serial program's bit for bit."""
    ln = schedule.dag_from_dict({"name": "ln_mm", "nodes": [
        {"name": "ln", "op": "layernorm", "engine": "aiv", "shape": {"rows": 4096, "cols": 2048}, "dtype": "bf16"},
        {"name": "mm", "op": "matmul", "engine": "aic", "shape": {"M": 4096, "K": 2048, "N": 2048}, "dtype": "bf16"}],
        "edges": [{"src": "ln", "dst": "mm", "kind": "data"}]})
    for tag, dag in (("fanout", workloads.mm_fanout(tmp_path, 2048, 1024, 2048)), ("ln_mm", ln),
                     ("chain2", workloads.e9_dag("e9_chain2", M=4096))):
        _, base = run(schedule.serial_schedule(dag), tmp_path, tag + "_serial", iters=1, warmup=0)
        r, outs = run(workloads.variants(dag, 4)["split"], tmp_path, "%s_p%d" % (tag, part), mode="graph_per_stream",
                      env={"KR_PLAN_PARTITION": str(part)})
        assert r["ok"] and r["gate_timeouts"] == 0, (tag, r)
        assert r["cu_partition_per_xcd"] == part and r["consumer_cus"] == 8 * part, r
        for node in base:
            assert np.array_equal(base[node], outs[node]), (tag, part, node)


def test_sync_micro_benchmark(gpu, tmp_path):
    """NHP_SYNC_BENCH (the reference's cross-stream sync micro-benchmark,
    exec/exec_main.cpp:751-833): 256 publish/wait kernel pairs per round on
    two hardware queues, without sync, with an event and with a device flag.
    Every flag wait is released (status 1); the result has the reference's
    keys."""
    import json
    out = tmp_path / "sync.json"
    os.environ["NHP_SYNC_BENCH"] = str(out)
    try:
        announce("plan_run NHP_SYNC_BENCH")
        rc = libapi.lib().kr_plan_run(b"unused", 1, 0, b"0", b"direct", str(tmp_path / "unused.json").encode())
    finally:
        del os.environ["NHP_SYNC_BENCH"]
    assert rc == 0
    r = json.loads(out.read_text())
    assert r["n"] == 256 and r["timeouts_flag"] == 0 and r["timeouts_event"] == 0 and r["timeouts_nosync"] == 0
    for k in ("us_per_pair_nosync", "us_per_pair_event", "us_per_pair_flag"):
        assert r[k] > 0
    announce("sync bench: %s" % json.dumps(r))
