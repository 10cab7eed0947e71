"""kr_qwen_run on the GPU: every mode produces bit-identical logits (the
relay split does not change any reduction), the last-token logits match the
fp32 CPU oracle (|d| <= 2e-2 + 1e-2|ref|) and its argmax."""

import os

import numpy as np
import pytest
import torch

from kernrelay_amd import libapi, modeldir
from oracle import qwen as oq
from tests.conftest import announce

pytestmark = pytest.mark.gpu

MODES = ["serial", "serial_fused", "serial_graph", "graph_whole", "relay_event", "relay_flag",
         "relay_flag_graph", "relay_split:1", "relay_split:2", "relay_split:4"]


def make(tmp, preset, seq, layers=None):
    d = modeldir.write_model_dir(tmp / preset, preset, seq=seq, layers=layers)
    ref = oq.write_reference(d)
    return d, ref


def run(d, mode, seq, dump=None, iters=2):
    if dump:
        os.environ["KR_DUMP_DIR"] = str(dump)
    try:
        announce("qwen_run %s mode=%s seq=%d" % (d.name, mode, seq))
        r = libapi.qwen_run(d, mode=mode, seq=seq, device=0, warmup=1, iters=iters)
    finally:
        os.environ.pop("KR_DUMP_DIR", None)
    assert r["_rc"] == 0, r
    return r


def check_logits(dump, ref, atol=2e-2):
    w = np.fromfile(dump / "last_logits_bf16.bin", dtype=np.uint16)
    g = torch.from_numpy(w.view(np.int16).copy()).view(torch.bfloat16).double()
    r = ref["last_logits"].double()
    err = (g - r).abs()
    assert bool((err <= atol + 1e-2 * r.abs()).all()), float(err.max())
    if ref["margin"] > 4e-2:
        assert int(g.argmax()) == ref["argmax"]


@pytest.mark.parametrize("preset", ["tiny-qwen2", "tiny-qwen3"])
def test_all_modes_bit_exact_and_match_oracle(gpu, tmp_path, preset):
    seq = 256
    d, ref = make(tmp_path, preset, seq)
    fnv = None
    for mode in MODES:
        dump = tmp_path / ("dump_" + mode.replace(":", "_"))
        dump.mkdir()
        r = run(d, mode, seq, dump)
        assert r["flag_timeouts"] == 0, (mode, r)
        assert r["ref_argmax"] == ref["argmax"]
        check_logits(dump, ref)
        if fnv is None:
            fnv = r["logits_fnv64"]
        assert r["logits_fnv64"] == fnv, (mode, r["logits_fnv64"], fnv)


def test_split_k_down_all_modes_bit_exact(gpu, tmp_path):
    """Layer shapes whose down projection splits K over idle CUs (I 8192 at
    seq 512: 4 output tiles of 128 K stages, eight pieces each; the gate/up
    projection never splits): every mode runs the same split (relay_flag
    releases its relay tile from the split's finishers), so the logits stay
    bit-identical across modes and match the oracle."""
    from kernrelay_amd import ops
    cfg = dict(modeldir.PRESETS["tiny-qwen3"])
    cfg["intermediate_size"] = 8192
    seq = 512
    assert ops.gemm_streamk_workspace(seq, cfg["hidden_size"], 8192)[0] > 0  # the down GEMM splits
    d = modeldir.write_model_dir(tmp_path / "splitk", cfg, seq=seq)
    ref = oq.write_reference(d)
    fnv = None
    os.environ["KR_QWEN_SPLITK"] = "1"
    try:
        for mode in MODES:
            dump = tmp_path / ("dump_" + mode.replace(":", "_"))
            dump.mkdir()
            r = run(d, mode, seq, dump)
            assert r["flag_timeouts"] == 0, (mode, r)
            check_logits(dump, ref)
            if fnv is None:
                fnv = r["logits_fnv64"]
            assert r["logits_fnv64"] == fnv, (mode, r["logits_fnv64"], fnv)
    finally:
        del os.environ["KR_QWEN_SPLITK"]


@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_epilogue_bit_exact(gpu, tmp_path, head_dim):
    """RoPE in the QKV GEMM's epilogue (models without q/k norms) gives the
    bits of the separate RoPE kernel: logits identical with and without it,
    serial and relay split, for head sizes 64 and 128, and the oracle's."""
    cfg = dict(modeldir.PRESETS["tiny-qwen2"])
    cfg.update(hidden_size=512, num_attention_heads=4, num_key_value_heads=2, head_dim=head_dim)
    seq = 512
    d = modeldir.write_model_dir(tmp_path / ("rope%d" % head_dim), cfg, seq=seq)
    ref = oq.write_reference(d)
    fnv = {}
    for epi in ("0", "1"):
        os.environ["KR_QWEN_ROPE_EPI"] = epi
        try:
            for mode in ("graph_whole", "relay_split:4"):
                dump = tmp_path / ("dump_%s_%s" % (epi, mode.replace(":", "_")))
                dump.mkdir()
                r = run(d, mode, seq, dump)
                check_logits(dump, ref)
                fnv[(epi, mode)] = r["logits_fnv64"]
        finally:
            del os.environ["KR_QWEN_ROPE_EPI"]
    assert len(set(fnv.values())) == 1, fnv


def test_qwen05_shapes_split_bit_exact(gpu, tmp_path):
    """Qwen2.5-0.5B layer shapes (H 896, 14/2 heads, D 64, I 4864, V 151936,
    tied) at seq 2048, two layers: serial == relay_split:4 (SwiGLU in the
    gate/up epilogue, and flag-released), oracle argmax. The logit bound's
    floor is 3e-2 here: the largest of 151936 bf16 logits' deviations from
    the fp32 oracle measured 0.0234 on MI355X whether the down projection
    splits K or not (mean 0.0039 both ways; 4 layers: 0.032 unsplit, 0.031
    split), one bf16 step away from the 2e-2 floor of the 2048-entry
    vocabularies."""
    seq = 2048
    d, ref = make(tmp_path, "qwen2.5-0.5b", seq, layers=2)
    dump = tmp_path / "dump"
    dump.mkdir()
    a = run(d, "graph_whole", seq, dump)
    check_logits(dump, ref, atol=3e-2)
    b = run(d, "relay_split:4", seq)
    assert a["logits_fnv64"] == b["logits_fnv64"]
    assert b["flag_timeouts"] == 0
    # the flag-released variant: SwiGLU workgroups appended to the gate/up
    # GEMM wait on its 4 row tiles
    os.environ["KR_SPLIT_SWIGLU"] = "flags"
    try:
        c = run(d, "relay_split:4", seq)
    finally:
        del os.environ["KR_SPLIT_SWIGLU"]
    assert a["logits_fnv64"] == c["logits_fnv64"]
    assert c["flag_timeouts"] == 0 and c["flag_edges"] > 0


def test_profile_many(gpu, tmp_path):
    d = modeldir.write_model_dir(tmp_path / "tiny", "tiny-qwen2", seq=256)
    ops = ["embedding", "rmsnorm", "add", "add_rmsnorm", "rope", "matmul_q", "matmul_k", "matmul_v",
           "attention", "matmul_o", "matmul_gate", "matmul_up", "silu", "mul", "swiglu", "matmul_down",
           "matmul_lm"]
    cases = [{"op": op, "k": k} for op in ops for k in (1, 2, 4)]
    announce("profile_many tiny")
    r = libapi.qwen_profile_many(d, cases, seq=256, device=0)
    assert r["_rc"] == 0, r
    got = {(c["op"], c["k"]) for c in r["cases"] if "best_us" in c}
    assert got == {(c["op"], c["k"]) for c in cases}
    assert all(c["best_us"] > 0 for c in r["cases"])
