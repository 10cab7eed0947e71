"""ctypes wrapper over libkernrelay.so's stable C ABI (include/kernrelay.h).

Same function names, argument order, result conventions and ``_rc`` field as
the reference's python/kernrelay/libapi.py:20-132, so callers written against
the reference keep working. Differences, all forced by the single-GPU target:

* default device is 0 (the reference defaults to its cluster's cards 6/7);
* ``qwen_pp_run`` / ``qwen_tp_run`` exist and bind, but the library answers
  ``{"error": "multi-GPU not in scope"}`` with ``_rc == 1``;
* ``plan_run`` accepts ``devices`` as a single id or a repeated one ("0,0").

The library location is ``$KERNRELAY_LIB`` or the in-tree build
``kernrelay_amd/lib/libkernrelay.so``; a missing library raises
FileNotFoundError (there is no fallback path).
"""

import ctypes
import json
import os
import tempfile
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_ROOT.parent

_LIB = None


def lib_path():
    env = os.environ.get("KERNRELAY_LIB")
    if env:
        return Path(env)
    return PACKAGE_ROOT / "lib" / "libkernrelay.so"


def lib():
    """Load libkernrelay.so once and declare every ABI signature."""
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not p.exists():
            raise FileNotFoundError(
                "%s does not exist; build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C kernrelay_amd/csrc`" % p)
        L = ctypes.CDLL(str(p))
        L.kr_version.restype = ctypes.c_char_p
        L.kr_version.argtypes = []
        L.kr_qwen_run.argtypes = [
            ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]
        L.kr_qwen_run.restype = ctypes.c_int
        L.kr_plan_run.argtypes = [
            ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
            ctypes.c_char_p, ctypes.c_char_p]
        L.kr_plan_run.restype = ctypes.c_int
        L.kr_qwen_pp_run.argtypes = [
            ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_char_p, ctypes.c_size_t]
        L.kr_qwen_pp_run.restype = ctypes.c_int
        L.kr_qwen_tp_run.argtypes = [
            ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_char_p, ctypes.c_size_t]
        L.kr_qwen_tp_run.restype = ctypes.c_int
        L.kr_qwen_profile_many.argtypes = [
            ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
            ctypes.c_char_p, ctypes.c_size_t]
        L.kr_qwen_profile_many.restype = ctypes.c_int
        _LIB = L
    return _LIB


def version():
    return lib().kr_version().decode()


def _payload(buf, rc):
    try:
        payload = json.loads(buf.value.decode())
    except Exception:
        payload = {"error": buf.value.decode(errors="replace")}
    payload["_rc"] = rc
    return payload


def qwen_run(model_dir, mode="serial_graph", seq=2048, device=0,
             warmup=1, iters=3):
    """Single-GPU prefill; see include/kernrelay.h for the mode list."""
    buf = ctypes.create_string_buffer(1 << 20)
    rc = lib().kr_qwen_run(
        str(model_dir).encode(), mode.encode(), int(seq), int(device),
        int(warmup), int(iters), buf, len(buf))
    return _payload(buf, rc)


def qwen_pp_run(model_dir, mode="pp", seq=2048, dev0=0, dev1=1,
                requests=2, warmup=1, iters=3):
    """Two-GPU pipeline parallel: not built on this target (rc 1)."""
    buf = ctypes.create_string_buffer(1 << 20)
    rc = lib().kr_qwen_pp_run(
        str(model_dir).encode(), mode.encode(), int(seq), int(dev0),
        int(dev1), int(requests), int(warmup), int(iters), buf, len(buf))
    return _payload(buf, rc)


def qwen_tp_run(model_dir, mode="tp2", seq=2048, dev0=0, dev1=1, tiles=2,
                warmup=1, iters=3):
    """Two-GPU tensor-parallel MLP: not built on this target (rc 1)."""
    buf = ctypes.create_string_buffer(1 << 20)
    rc = lib().kr_qwen_tp_run(
        str(model_dir).encode(), mode.encode(), int(seq), int(dev0), int(dev1),
        int(tiles), int(warmup), int(iters), buf, len(buf))
    return _payload(buf, rc)


def plan_run(schedule_json, devices="0", mode="direct", iters=3, warmup=1,
             out_json=None):
    """Run one schedule.json; returns the result file's JSON plus ``_rc``."""
    out = Path(out_json) if out_json else Path(
        tempfile.mkstemp(prefix="kr_plan_", suffix=".json")[1])
    rc = lib().kr_plan_run(
        str(schedule_json).encode(), int(iters), int(warmup),
        str(devices).encode(), mode.encode(), str(out).encode())
    try:
        payload = json.loads(out.read_text(encoding="utf-8"))
    except Exception:
        payload = {"error": "no result", "rc": rc, "out": str(out)}
    payload["_rc"] = rc
    return payload


def qwen_profile_many(model_dir, cases, seq=2048, device=0):
    """cases: [{"op":..., "k":...}] -> dict; weights loaded once."""
    fd, path = tempfile.mkstemp(prefix="kr_profile_", suffix=".json")
    os.close(fd)
    try:
        Path(path).write_text(json.dumps({"cases": cases}), encoding="utf-8")
        buf = ctypes.create_string_buffer(4 << 20)
        rc = lib().kr_qwen_profile_many(
            str(model_dir).encode(), path.encode(), int(seq), int(device),
            buf, len(buf))
        return _payload(buf, rc)
    finally:
        os.unlink(path)
