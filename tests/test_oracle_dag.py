"""Pin the DAG-input oracle against the reference's own recorded results.

results/final/e34_raw.json holds the reference executor's checksums for its
E3/E4 DAGs (fp16, 2 ranks, DetValue inputs): mm->gelu 0.84616 (:15),
mm->softmax 7.714923 (:2301), mm->{gelu,softmax} 8.846179 (:2969) and
mm->cast 7405.689026 and LayerNorm->mm 5.91964 (:2003). The oracle
restatement must reproduce them; a wrong seed, input role, row order or op
(e.g. an unbiased variance or eps 1e-6 in the LayerNorm) fails here.
"""

import numpy as np
import pytest

from kernrelay_amd import schedule, workloads
from oracle import dag_eval, dag_inputs


def ref_dag(name, consumers):
    """The reference's dags/f01_mm_gelu_c2.json, e3_mm_softmax.json,
    e3_mm_cast.json and f04_mm_fanout_c2.json shapes (M=32768, K=1024, N=2048, fp16)."""
    return workloads.e34_dag(name, consumers)


KATS = [
    ("f01_mm_gelu_c2", ["gelu"], 0.84616),
    ("e3_mm_softmax", ["softmax"], 7.714923),
    ("f04_mm_fanout_c2", ["gelu", "softmax"], 8.846179),
    ("e3_mm_cast", ["cast"], 7405.689026),
    ("e3_ln_mm", None, 5.91964),
]


def ln_mm_dag():
    """The reference's dags/e3_ln_mm.json: a LayerNorm producer on the vector
    engine feeding a GEMM consumer (the reverse edge), 32768 x 2048, fp16;
    its recorded checksum is results/final/e34_raw.json:2003 (5.91964)."""
    return workloads.e34_dag("e3_ln_mm", None)


def kat_dag(name, consumers):
    return ln_mm_dag() if consumers is None else ref_dag(name, consumers)


# The reference's two-wave DAGs on one device (results/final/e9_raw.json:
# the same checksum for serial, B0 and the split at k = 4 and 8; fp16, 2
# ranks, DetValue inputs), with the bound each is held to. e9_chain2's
# second GEMM reads GELU outputs over K = 2048: the oracle's checksum
# (1.6084236, unchanged with fp64 accumulation) sits 1.2e-5 from the
# recorded 1.608412 — one fp16 rounding step of a value near 0.02 among the
# 32768 words summed, the reference's closed fp16 GEMM rounding a product
# the other way. A wrong edge moves it by far more (mm2 reading mm1's
# output: 2.474; mm2 on its own inputs: 5.663; one rank: 0.273).
E9_KATS = [
    ("e9_two_waves", 3.429432, 1.5e-6),
    ("e9_chain2", 1.608412, 2e-5),
]


@pytest.mark.parametrize("name,consumers,expected", KATS)
def test_reference_checksums(name, consumers, expected):
    dag = kat_dag(name, consumers)
    sched = schedule.build_fixed_schedule(dag, {n.name: 4 for n in dag.nodes}, nranks=2)
    got = dag_eval.checksum(sched)
    # the reference prints 7 significant digits and computes with closed
    # aclnn kernels; its own consistency gate is rtol 1e-3 (stats.py:3)
    assert abs(got - expected) <= 2e-6 * abs(expected) + 1e-5, (name, got, expected)


def test_checksum_independent_of_split():
    dag = ref_dag("f04_mm_fanout_c2", ["gelu", "softmax"])
    a = dag_eval.checksum(schedule.serial_schedule(dag, nranks=2))
    b = dag_eval.checksum(schedule.build_fixed_schedule(dag, {"mm": 8, "gelu": 4, "softmax": 2}, nranks=2))
    assert a == b


def test_det_values_range_and_grid():
    v = dag_inputs.det_values(12345, 100000, dtype=None)
    assert v.min() >= -11 / 256 and v.max() <= 11 / 256
    assert np.all(np.round(v * 256) == v * 256)
    # 23 distinct levels, each present
    assert len(np.unique(v)) == 23


def test_det_values_known_answers():
    # hand-computed: seed 0, i = 0 -> h = 7 -> (7 >> 8) % 23 = 0 -> -11/256
    assert dag_inputs.det_values(0, 1, dtype=None)[0] == -11 / 256
    # i = 1 -> h = 2654435761 + 7 = 2654435768 -> >> 8 = 10368889 = 23*450821 + 6 -> -5/256
    assert 2654435768 >> 8 == 10368889 and 10368889 == 23 * 450821 + 6
    assert dag_inputs.det_values(0, 2, dtype=None)[1] == -5 / 256
    # seed wraps mod 2^32: seed*40503 is taken mod 2^32 before the add
    big = 0xFFFFFFFF
    h = (0 * 2654435761 + (big * 40503) + 7) & 0xFFFFFFFF
    assert dag_inputs.det_values(big, 1, dtype=None)[0] == (((h >> 8) % 23) - 11) / 256


def test_node_seed_fnv():
    # FNV-1a 32-bit of "a" is 0xe40c292c (published test vector)
    assert dag_inputs.fnv1a("a") == 0xE40C292C
    assert dag_inputs.node_seed("a", 1) == (0xE40C292C + 7919) & 0xFFFFFFFF


def test_bf16_rounding_helper():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3e38, np.inf], dtype=np.float32)
    bits = dag_inputs.f32_to_bf16_bits(x)
    back = dag_inputs.bf16_bits_to_f32(bits)
    # ties to even: 1 + 2^-8 -> 1.0, 1 + 3*2^-8 -> 1 + 2^-6
    assert back[0] == 1.0 and back[1] == 1.0 and back[2] == 1.0 + 2 ** -6
    assert back[3] == -2.5 and np.isinf(back[5])


@pytest.mark.parametrize("name,expected,tol", E9_KATS)
def test_e9_reference_checksums(name, expected, tol):
    """Two independent mm -> GELU chains, and mm -> GELU -> mm -> GELU (a GEMM
    consuming a GELU producer's rows), split at k=4 over 2 ranks, reproduce
    the reference's recorded checksums."""
    dag = workloads.e9_dag(name)
    sched = schedule.build_fixed_schedule(dag, {n.name: 4 for n in dag.nodes}, nranks=2)
    got = dag_eval.checksum(sched)
    assert abs(got - expected) <= tol, (name, got, expected)
    assert dag_eval.checksum(schedule.serial_schedule(dag, nranks=2)) == got
