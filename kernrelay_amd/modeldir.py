"""Synthetic model directories in the reference's export format.

Writes what scripts/export_model.py:116-226 writes for a real checkpoint —
manifest.json (config, tensors{name: offset, bytes, dtype, shape}, seq, seed,
max_pos), weights.bin (bf16; matmul weights transposed to weight_t [K, N]),
ids.bin (int64 [seq]) — from random-init weights, since no checkpoint can be
fetched here. Tensor names and write order are the reference's
(export_model.py:171-204).

Init (seeded): projection weights, biases and embeddings ~ N(0, 0.02);
RMSNorm gains 1 + N(0, 0.02) (HF initialises gains to 1; the small spread
makes a dropped or transposed gain visible to the parity tests); RoPE tables
from export_model.py:70-77; token ids uniform in [0, vocab).

The reference-logit files (ref_last_logits.bin, ref.json) come from the
oracle, not from here.
"""

import json
from pathlib import Path

import torch

PRESETS = {
    # Qwen2.5-0.5B shapes (tied lm_head)
    "qwen2.5-0.5b": dict(hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
                         num_attention_heads=14, num_key_value_heads=2, head_dim=64, vocab_size=151936,
                         tie_word_embeddings=True, attention_bias=True, qk_norm=False,
                         rope_theta=1e6, rms_norm_eps=1e-6),
    # Qwen2.5-7B shapes (the benchmarked prefill)
    "qwen2.5-7b": dict(hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                       num_attention_heads=28, num_key_value_heads=4, head_dim=128, vocab_size=152064,
                       tie_word_embeddings=False, attention_bias=True, qk_norm=False,
                       rope_theta=1e6, rms_norm_eps=1e-6),
    # Qwen3-8B text shapes (the Qwen3-VL-8B language model)
    "qwen3-8b": dict(hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                     num_attention_heads=32, num_key_value_heads=8, head_dim=128, vocab_size=151936,
                     tie_word_embeddings=False, attention_bias=False, qk_norm=True,
                     rope_theta=1e6, rms_norm_eps=1e-6),
    # small shapes for the parity tests
    "tiny-qwen2": dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=1024,
                       tie_word_embeddings=True, attention_bias=True, qk_norm=False,
                       rope_theta=1e6, rms_norm_eps=1e-6),
    "tiny-qwen3": dict(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=128, vocab_size=2048,
                       tie_word_embeddings=False, attention_bias=False, qk_norm=True,
                       rope_theta=1e6, rms_norm_eps=1e-6),
}


def rope_table(max_pos, D, theta):
    """[1, 1, max_pos, D] bf16 cos/sin as export_model.py:70-77 builds them."""
    inv = 1.0 / (torch.tensor(theta, dtype=torch.float64) ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    pos = torch.arange(max_pos, dtype=torch.float64)
    freqs = torch.outer(pos, inv)
    cos = torch.cat([freqs.cos(), freqs.cos()], dim=-1).to(torch.bfloat16)
    sin = torch.cat([freqs.sin(), freqs.sin()], dim=-1).to(torch.bfloat16)
    return cos.reshape(1, 1, max_pos, D), sin.reshape(1, 1, max_pos, D)


class _Writer:
    def __init__(self, path):
        self.f = open(path, "wb")
        self.cursor = 0
        self.tensors = {}

    def put(self, name, t, source_shape=None):
        t = t.detach().contiguous()
        dtype = str(t.dtype).replace("torch.", "")
        data = t.view(torch.int16).cpu().numpy().tobytes() if t.dtype == torch.bfloat16 else t.cpu().numpy().tobytes()
        self.tensors[name] = {"offset": self.cursor, "bytes": len(data), "dtype": dtype, "shape": list(t.shape)}
        if source_shape is not None:
            self.tensors[name]["source_shape"] = list(source_shape)
        self.f.write(data)
        self.cursor += len(data)

    def close(self):
        self.f.close()


def write_model_dir(out_dir, preset_or_config, seq=2048, seed=1234, max_pos=None, layers=None,
                    device=None, std=0.02, gain_std=None):
    """Write a random-init model directory; returns its Path.

    preset_or_config: a PRESETS key or a config dict with the same keys.
    layers: override num_hidden_layers (short stacks for tests).
    device: torch device for weight generation ("cuda" generates on the GPU,
    which is much faster for the 7B/8B presets); values are the file's.
    gain_std: spread of the RMSNorm gains around 1 (default: std); a wide
    spread makes a misplaced or dropped gain stand out in a comparison.
    """
    gain_std = std if gain_std is None else gain_std
    cfg = dict(PRESETS[preset_or_config]) if isinstance(preset_or_config, str) else dict(preset_or_config)
    if layers is not None:
        cfg["num_hidden_layers"] = int(layers)
    H, I, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    HQ, HKV, V = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["vocab_size"]
    D = cfg.get("head_dim", H // HQ)
    max_pos = max_pos or max(4096, seq)
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    dev = torch.device(device or "cpu")
    gen = torch.Generator(device=dev).manual_seed(seed)

    def normal(*shape, mean=0.0, sd=None):
        t = torch.empty(*shape, dtype=torch.float32, device=dev).normal_(mean, std if sd is None else sd,
                                                                          generator=gen)
        return t.to(torch.bfloat16).cpu()

    w = _Writer(out / "weights.bin")
    for l in range(L):
        p = "L%02d." % l
        for role, (k, n) in (("q_proj", (H, HQ * D)), ("k_proj", (H, HKV * D)), ("v_proj", (H, HKV * D)),
                             ("o_proj", (HQ * D, H))):
            w.put(p + role + ".weight_t", normal(k, n), source_shape=(n, k))
        if cfg.get("attention_bias", False):
            for role, n in (("q_proj", HQ * D), ("k_proj", HKV * D), ("v_proj", HKV * D)):
                w.put(p + role + ".bias", normal(n))
        for role, (k, n) in (("gate_proj", (H, I)), ("up_proj", (H, I)), ("down_proj", (I, H))):
            w.put(p + role + ".weight_t", normal(k, n), source_shape=(n, k))
        for role in ("input_layernorm", "post_attention_layernorm"):
            w.put(p + role + ".weight", normal(H, mean=1.0, sd=gain_std))
        if cfg.get("qk_norm", False):
            for role in ("q_norm", "k_norm"):
                w.put(p + role + ".weight", normal(D, mean=1.0, sd=gain_std))
    emb = normal(V, H)
    w.put("embed.weight", emb)
    lm = emb if cfg.get("tie_word_embeddings", True) else normal(V, H)
    w.put("lm_head.weight_t", lm.t().contiguous(), source_shape=(V, H))
    w.put("final_norm.weight", normal(H, mean=1.0, sd=gain_std))
    cos, sin = rope_table(max_pos, D, cfg.get("rope_theta", 1e6))
    w.put("rope.cos", cos)
    w.put("rope.sin", sin)
    w.close()

    ids = torch.randint(0, V, (1, seq), generator=torch.Generator().manual_seed(seed), dtype=torch.long)
    ids.numpy().tofile(out / "ids.bin")
    manifest = {
        "config": {
            "arch": "qwen3_vl" if cfg.get("qk_norm") else "qwen2.5", "hidden_size": H,
            "intermediate_size": I, "num_hidden_layers": L, "num_attention_heads": HQ,
            "num_key_value_heads": HKV, "head_dim": D, "vocab_size": V,
            "rms_norm_eps": cfg.get("rms_norm_eps", 1e-6), "qk_norm": bool(cfg.get("qk_norm", False)),
            "attention_bias": bool(cfg.get("attention_bias", False)),
            "tie_word_embeddings": bool(cfg.get("tie_word_embeddings", True)),
            "rope_theta": cfg.get("rope_theta", 1e6), "hidden_act": "silu",
        },
        "tensors": w.tensors, "seq": seq, "seed": seed, "max_pos": max_pos,
        "init": {"kind": "normal", "std": std, "norm_gain_mean": 1.0, "norm_gain_std": gain_std},
    }
    (out / "manifest.json").write_text(json.dumps(manifest, indent=1))
    return out


def model_flops(cfg, seq):
    """Algorithmic prefill FLOPs: 2*M*N*K per GEMM, causal attention counted
    as half (2*2*S(S+1)/2*HQ*D per layer), lm_head over all rows."""
    H, I, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    HQ, HKV, V = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["vocab_size"]
    D = cfg.get("head_dim", H // HQ)
    S = seq
    per_layer = 2 * S * H * (HQ + 2 * HKV) * D + 2 * S * HQ * D * H + 2 * S * H * 2 * I + 2 * S * I * H
    attn = 2 * 2 * (S * (S + 1) / 2) * HQ * D
    return L * (per_layer + attn) + 2 * S * H * V


def model_gemm_flops(cfg, seq):
    H, I, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    HQ, HKV, V = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["vocab_size"]
    D = cfg.get("head_dim", H // HQ)
    S = seq
    per_layer = 2 * S * H * (HQ + 2 * HKV) * D + 2 * S * HQ * D * H + 2 * S * H * 2 * I + 2 * S * I * H
    return L * per_layer + 2 * S * H * V
