"""Qwen2.5 / Qwen3-text prefill oracle over a model directory — test
infrastructure only.

Op order of the reference's BuildSerial (exec/qwen_main.cpp:925-992) with
EmitQkv (:1336-1344) and EmitQkNorm (:1346-1357); weight layout and tensor
names of scripts/export_model.py:142-204 (matmul weights stored as weight_t
[K, N]). Every stored activation is rounded to bf16 (oracle/ops.py); the
residual stream alternates h0/h1 exactly as the reference's buffers do.

Pinned against transformers' Qwen2ForCausalLM / Qwen3ForCausalLM built from
a local config and loaded with the same model directory
(oracle/hf_reference.py), at tiny shapes covering QKV bias + GQA + tied
lm_head and q/k-norm + untied lm_head (tests/test_oracle_qwen.py): last-row
logits within 2e-2 + 1e-2|ref| at the default init and within 3e-2 max|ref|
at a wide init, the same argmax, and nine planted composition mistakes
(residual, bias, RoPE sign or skip, GQA mapping, scale, gate/up order, norm
gain, eps) each rejected by more than 10x that bound.
"""

import json
from pathlib import Path

import numpy as np
import torch

from . import ops

F32 = torch.float32


class ModelDir:
    """Read-only view of manifest.json + weights.bin + ids.bin."""

    def __init__(self, path):
        self.path = Path(path)
        self.manifest = json.loads((self.path / "manifest.json").read_text())
        c = self.manifest["config"]
        self.H = int(c["hidden_size"])
        self.I = int(c["intermediate_size"])
        self.L = int(c["num_hidden_layers"])
        self.HQ = int(c["num_attention_heads"])
        self.HKV = int(c["num_key_value_heads"])
        self.V = int(c["vocab_size"])
        self.D = int(c.get("head_dim", self.H // self.HQ))
        self.eps = float(c.get("rms_norm_eps", 1e-6))
        self.qk_norm = bool(c.get("qk_norm", False))
        self.bias = bool(c.get("attention_bias", True)) and "L00.q_proj.bias" in self.manifest["tensors"]
        self.seq = int(self.manifest["seq"])
        self._raw = np.memmap(self.path / "weights.bin", dtype=np.uint8, mode="r")

    def tensor(self, name):
        """bf16 tensor (as fp32 values) named `name` in its manifest shape."""
        t = self.manifest["tensors"][name]
        raw = np.asarray(self._raw[t["offset"]: t["offset"] + t["bytes"]]).view(np.int16)
        return torch.from_numpy(raw.copy()).view(torch.bfloat16).reshape(t["shape"]).to(F32)

    def ids(self):
        return torch.from_numpy(np.fromfile(self.path / "ids.bin", dtype=np.int64))

    def rope(self, S):
        D = self.D
        cos = self.tensor("rope.cos").reshape(-1, D)[:S]
        sin = self.tensor("rope.sin").reshape(-1, D)[:S]
        return cos, sin


def layer_forward(m, l, h, x, cos, sin, p_dt=None):
    """One decoder layer. h = residual stream (bf16 values), x = normed input.
    Returns (h_next, x_next_unnormed_sum) where the caller applies the next norm.
    p_dt: attention's P rounded to this type before P.V (ops.attention)."""
    S = x.shape[0]
    p = "L%02d." % l
    HQ, HKV, D = m.HQ, m.HKV, m.D
    bq = m.tensor(p + "q_proj.bias") if m.bias else None
    bk = m.tensor(p + "k_proj.bias") if m.bias else None
    bv = m.tensor(p + "v_proj.bias") if m.bias else None
    q = ops.gemm(x, m.tensor(p + "q_proj.weight_t"), bq).reshape(S, HQ, D)
    k = ops.gemm(x, m.tensor(p + "k_proj.weight_t"), bk).reshape(S, HKV, D)
    v = ops.gemm(x, m.tensor(p + "v_proj.weight_t"), bv).reshape(S, HKV, D)
    if m.qk_norm:
        q, _ = ops.rmsnorm(q, m.tensor(p + "q_norm.weight"), m.eps)
        k, _ = ops.rmsnorm(k, m.tensor(p + "k_norm.weight"), m.eps)
    q = ops.rope(q, cos, sin)
    k = ops.rope(k, cos, sin)
    a = ops.attention(q, k, v, p_dt=p_dt).reshape(S, HQ * D)
    o = ops.gemm(a, m.tensor(p + "o_proj.weight_t"))
    x2, h2, _ = ops.add_rmsnorm(h, o, m.tensor(p + "post_attention_layernorm.weight"), m.eps)
    g = ops.gemm(x2, m.tensor(p + "gate_proj.weight_t"))
    u = ops.gemm(x2, m.tensor(p + "up_proj.weight_t"))
    act = ops.swiglu(g, u)
    d = ops.gemm(act, m.tensor(p + "down_proj.weight_t"))
    return h2, d


def prefill(model_dir, layers=None, threads=None, lm_all_rows=False, p_dt=None):
    """Run the prefill; returns dict(last_logits=fp32 [V] of bf16 values,
    argmax, margin, and argmax_fp32 / margin_fp32 of the last row's product
    before its bf16 rounding, where top logits can tie). `layers` truncates
    the stack (tests of the CPU cost).
    lm_all_rows: compute the lm_head over every row, as the reference's
    prefill does (qwen_main.cpp:920, :989), instead of the last row only
    (the work of a timed baseline; the last row then differs from the
    one-row product only by fp32 summation order). p_dt: attention's P
    rounded to this type before P.V, as a 16-bit matrix unit computes it
    (ops.attention)."""
    if threads:
        torch.set_num_threads(threads)
    m = model_dir if isinstance(model_dir, ModelDir) else ModelDir(model_dir)
    ids = m.ids()
    S = ids.numel()
    cos, sin = m.rope(S)
    with torch.no_grad():
        h = ops.embedding(m.tensor("embed.weight"), ids)
        x, _ = ops.rmsnorm(h, m.tensor("L00.input_layernorm.weight"), m.eps)
        L = m.L if layers is None else layers
        for l in range(L):
            h2, d = layer_forward(m, l, h, x, cos, sin, p_dt=p_dt)
            gname = ("L%02d.input_layernorm.weight" % (l + 1)) if l + 1 < L else "final_norm.weight"
            x, h, _ = ops.add_rmsnorm(h2, d, m.tensor(gname), m.eps)
        logits = ops.gemm(x if lm_all_rows else x[-1:], m.tensor("lm_head.weight_t"))[-1]
        l32 = ops.gemm(x[-1:], m.tensor("lm_head.weight_t"), dt=torch.float32)[-1]
    top, top32 = torch.topk(logits, 2), torch.topk(l32, 2)
    return {"last_logits": logits, "argmax": int(top.indices[0]),
            "margin": float(top.values[0] - top.values[1]),
            "argmax_fp32": int(top32.indices[0]), "margin_fp32": float(top32.values[0] - top32.values[1])}


def write_reference(model_dir, result=None, layers=None):
    """Write ref_last_logits.bin (fp32 [V]) and ref.json for kr_qwen_run's
    Verify (the files export_model.py writes from HF logits, :211-226)."""
    res = result if result is not None else prefill(model_dir, layers=layers)
    path = Path(model_dir.path if isinstance(model_dir, ModelDir) else model_dir)
    res["last_logits"].numpy().astype(np.float32).tofile(path / "ref_last_logits.bin")
    last = res["last_logits"]
    ref = {"argmax_last": res["argmax"], "sum": float(last.sum()), "abs_mean": float(last.abs().mean()),
           "margin": res["margin"], "source": "oracle fp32 CPU"}
    (path / "ref.json").write_text(json.dumps(ref, indent=1))
    return res
