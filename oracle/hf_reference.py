"""Independent reference logits from transformers — test infrastructure only.

The reference's exporter runs the Hugging Face model on the model directory's
own checkpoint and writes its last-token logits as ref_last_logits.bin (fp32
[V]) and ref.json (argmax_last, sum, abs_mean) for the runtime's Verify
(scripts/export_model.py:205-223). No checkpoint can be fetched here, so this
module builds transformers' Qwen2ForCausalLM / Qwen3ForCausalLM from a local
config object (no network: the config is constructed, never downloaded),
loads the synthetic model directory's weights into it (each weight_t [K, N]
transposed back to the checkpoint's [N, K]), and runs the prefill on the CPU.

It shares no code with oracle/qwen.py: the layer composition (residual order,
q/k-norm placement, bias before RoPE, GQA head mapping, SwiGLU, tied or untied
lm_head) is transformers' own, which is what pins the oracle's composition
(tests/test_oracle_qwen.py).

Differences from the reference's exporter, by design:
  * dtype: fp32 by default (the exporter used bf16 on its device); bf16 is
    available for a like-for-like run;
  * RoPE: transformers computes cos/sin in fp32 from its own inverse
    frequencies, while the model directory stores bf16 tables
    (export_model.py:70-77) that the runtime uses; the two differ by at most
    one bf16 rounding of each table entry.
"""

import json
from pathlib import Path

import numpy as np
import torch


def _manifest(model_dir):
    return json.loads((Path(model_dir) / "manifest.json").read_text())


def _tensor(raw, meta, name):
    t = meta["tensors"][name]
    b = np.asarray(raw[t["offset"]: t["offset"] + t["bytes"]]).view(np.int16).copy()
    return torch.from_numpy(b).view(torch.bfloat16).reshape(t["shape"])


def hf_config(model_dir):
    """transformers config for the model directory's manifest (constructed
    locally; nothing is fetched)."""
    meta = _manifest(model_dir)
    c = meta["config"]
    common = dict(vocab_size=int(c["vocab_size"]), hidden_size=int(c["hidden_size"]),
                  intermediate_size=int(c["intermediate_size"]),
                  num_hidden_layers=int(c["num_hidden_layers"]),
                  num_attention_heads=int(c["num_attention_heads"]),
                  num_key_value_heads=int(c["num_key_value_heads"]),
                  head_dim=int(c["head_dim"]), max_position_embeddings=int(meta.get("max_pos", 4096)),
                  rope_theta=float(c.get("rope_theta", 1e6)), rms_norm_eps=float(c.get("rms_norm_eps", 1e-6)),
                  tie_word_embeddings=bool(c.get("tie_word_embeddings", True)), hidden_act="silu",
                  attention_dropout=0.0)
    if c.get("qk_norm"):
        from transformers import Qwen3Config
        return Qwen3Config(attention_bias=bool(c.get("attention_bias", False)), **common), "qwen3"
    from transformers import Qwen2Config
    return Qwen2Config(**common), "qwen2"


def hf_model(model_dir, dtype=torch.float32, device="cpu"):
    """transformers Qwen2/Qwen3ForCausalLM holding the model directory's
    weights, built on `device` (a GPU builds a 7B model in seconds)."""
    cfg, kind = hf_config(model_dir)
    if kind == "qwen3":
        from transformers import Qwen3ForCausalLM as Cls
    else:
        from transformers import Qwen2ForCausalLM as Cls
    cfg._attn_implementation = "eager"
    with torch.device(device):
        model = Cls(cfg).eval()
    meta = _manifest(model_dir)
    raw = np.memmap(Path(model_dir) / "weights.bin", dtype=np.uint8, mode="r")
    sd = {}
    c = meta["config"]
    for l in range(int(c["num_hidden_layers"])):
        p, q = "L%02d." % l, "model.layers.%d." % l
        for role in ("q_proj", "k_proj", "v_proj", "o_proj"):
            sd[q + "self_attn." + role + ".weight"] = _tensor(raw, meta, p + role + ".weight_t").t()
        for role in ("q_proj", "k_proj", "v_proj"):
            if (p + role + ".bias") in meta["tensors"]:
                sd[q + "self_attn." + role + ".bias"] = _tensor(raw, meta, p + role + ".bias")
        for role in ("gate_proj", "up_proj", "down_proj"):
            sd[q + "mlp." + role + ".weight"] = _tensor(raw, meta, p + role + ".weight_t").t()
        for role in ("input_layernorm", "post_attention_layernorm"):
            sd[q + role + ".weight"] = _tensor(raw, meta, p + role + ".weight")
        if c.get("qk_norm"):
            for role in ("q_norm", "k_norm"):
                sd[q + "self_attn." + role + ".weight"] = _tensor(raw, meta, p + role + ".weight")
    sd["model.embed_tokens.weight"] = _tensor(raw, meta, "embed.weight")
    sd["model.norm.weight"] = _tensor(raw, meta, "final_norm.weight")
    if not cfg.tie_word_embeddings:
        sd["lm_head.weight"] = _tensor(raw, meta, "lm_head.weight_t").t()
    sd = {k: v.to(device=device, dtype=dtype).contiguous() for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if not (cfg.tie_word_embeddings and m == "lm_head.weight")]
    if missing or unexpected:
        raise RuntimeError("weights do not fit the transformers model: missing %s, unexpected %s"
                           % (missing, unexpected))
    if cfg.tie_word_embeddings:
        model.tie_weights()
    return model.to(dtype)


def last_logits(model_dir, dtype=torch.float32, threads=None, device="cpu"):
    """fp32 [V] last-token logits (on the CPU) of the transformers model on
    ids.bin, run on `device`. On a GPU keep dtype fp32: the eager attention
    multiplies by a transposed key view, which this stack runs reliably in
    fp32 only."""
    if threads:
        torch.set_num_threads(threads)
    ids = torch.from_numpy(np.fromfile(Path(model_dir) / "ids.bin", dtype=np.int64)).reshape(1, -1)
    model = hf_model(model_dir, dtype, device)
    with torch.no_grad():
        out = model(input_ids=ids.to(device), use_cache=False, logits_to_keep=1)
    last = out.logits[0, -1].float().cpu()
    del model, out
    return last


def write_reference(model_dir, dtype=torch.float32, device="cpu"):
    """Write ref_last_logits.bin and ref.json from transformers run on
    `device` (the files export_model.py:211-223 writes, which kr_qwen_run's
    Verify compares against); returns the logits and their top-2."""
    last = last_logits(model_dir, dtype, device=device)
    path = Path(model_dir)
    last.numpy().astype(np.float32).tofile(path / "ref_last_logits.bin")
    top = torch.topk(last, 2)
    where = "GPU" if str(device).startswith("cuda") else "CPU"
    ref = {"argmax_last": int(top.indices[0]), "sum": float(last.sum()), "abs_mean": float(last.abs().mean()),
           "margin": float(top.values[0] - top.values[1]),
           "source": "transformers %s %s %s" % (hf_config(path)[1], str(dtype).replace("torch.", ""), where)}
    (path / "ref.json").write_text(json.dumps(ref, indent=1))
    return {"last_logits": last, "argmax": ref["argmax_last"], "margin": ref["margin"]}


def main(argv=None):
    """python -m oracle.hf_reference MODEL_DIR [--device cuda] [--dtype bf16]:
    the reference step of the exporter for a model directory."""
    import argparse
    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("model_dir")
    ap.add_argument("--device", default="cpu")
    ap.add_argument("--dtype", choices=("fp32", "bf16"), default="fp32")
    args = ap.parse_args(argv)
    r = write_reference(args.model_dir, torch.float32 if args.dtype == "fp32" else torch.bfloat16, args.device)
    print(json.dumps({"argmax_last": r["argmax"], "margin": r["margin"]}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
