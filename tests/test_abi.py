"""The C-ABI library loads and exports every entry point include/*.h declares;
error conventions and schedule rejection behave as the reference's (no GPU)."""

import json
import re
import subprocess
import sys
from pathlib import Path

import pytest

from kernrelay_amd import libapi, schedule, workloads

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(kr_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_headers_declare_the_reference_abi():
    names = declared_functions()
    # the six reference entry points (reference include/kernrelay.h:11-69)
    for n in ("kr_version", "kr_plan_run", "kr_qwen_run", "kr_qwen_pp_run", "kr_qwen_tp_run",
              "kr_qwen_profile_many"):
        assert n in names


def test_library_exports_every_declared_symbol():
    L = libapi.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_version():
    assert "KernRelay" in libapi.version()


@pytest.mark.parametrize("fn", ["qwen_pp_run", "qwen_tp_run"])
def test_multi_gpu_entries_report_out_of_scope(fn):
    r = getattr(libapi, fn)("/nonexistent")
    assert r["_rc"] == 1 and "multi-GPU not in scope" in r["error"]


def test_qwen_run_errors_into_json():
    r = libapi.qwen_run("", mode="serial")
    assert r["_rc"] == 1 and "model path required" in r["error"]
    r = libapi.qwen_run("/nonexistent", mode="pp")
    assert r["_rc"] == 1


def test_qwen_run_small_buffer():
    import ctypes
    buf = ctypes.create_string_buffer(8)
    rc = libapi.lib().kr_qwen_run(b"", b"serial", 16, 0, 0, 1, buf, len(buf))
    assert rc == 1  # error JSON truncated into the tiny buffer, never overflowed
    assert len(buf.value) < 8


def test_plan_run_null_args():
    assert libapi.lib().kr_plan_run(None, 1, 0, None, None, None) == 2


def run_plan_subprocess(path, mode="direct"):
    code = ("import sys; sys.path.insert(0, %r); from kernrelay_amd import libapi; "
            "r = libapi.plan_run(%r, devices='0', mode=%r, iters=1, warmup=0); print('RC', r['_rc'])"
            % (str(ROOT), str(path), mode))
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)


def test_invalid_schedules_rejected_with_reference_markers(tmp_path):
    """E0 gate (reference python/kernrelay/e0.py:98-108): every broken schedule
    exits non-zero, writes no result and names its marker on stderr."""
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, {"mm": 2, "gelu": 2})
    variants = schedule.invalid_variants(sched)
    assert set(variants) == {"duplicate_engine", "ghost_task", "wait_cycle", "row_overflow"}
    for label, (bad, marker) in variants.items():
        p = schedule.dump_schedule(bad, tmp_path / (label + ".json"))
        proc = run_plan_subprocess(p)
        assert "RC 1" in proc.stdout, (label, proc.stdout, proc.stderr)
        assert marker in proc.stderr, (label, proc.stderr)


def test_unknown_op_and_mode_rejected(tmp_path):
    dag = workloads.tiny_mm_gelu(tmp_path)
    sched = schedule.build_fixed_schedule(dag, {})
    bad = json.loads(json.dumps(sched))
    bad["nodes"][1]["op"] = "topk"
    proc = run_plan_subprocess(schedule.dump_schedule(bad, tmp_path / "topk.json"))
    assert "RC 1" in proc.stdout and "not built" in proc.stderr
    proc = run_plan_subprocess(schedule.dump_schedule(sched, tmp_path / "ok.json"), mode="graph_bogus")
    assert "RC 1" in proc.stdout and "not built" in proc.stderr


def test_gemm_add_rmsnorm_rejects_strided_views():
    """The C entry takes C, res, y and sum as packed [M, N] rows: a strided
    view is refused before anything reaches the library."""
    import torch

    from kernrelay_amd import ops

    M, N, K = 64, 256, 64
    A = torch.zeros(M, K, dtype=torch.bfloat16)
    Bt = torch.zeros(N, K, dtype=torch.bfloat16)
    wide = torch.zeros(M, N + 8, dtype=torch.bfloat16)
    packed = torch.zeros(M, N, dtype=torch.bfloat16)
    gamma = torch.ones(N, dtype=torch.bfloat16)
    pub = ops.KrPub(None, 0, M, 0)
    for bad in ("C", "res", "y", "sum_out"):
        args = {"C": packed, "res": packed, "y": packed, "sum_out": packed}
        args[bad] = wide[:, :N]
        with pytest.raises(ValueError, match=bad):
            ops.gemm_add_rmsnorm(A, Bt, args["C"], args["res"], gamma, args["y"], pub, sum_out=args["sum_out"])
