"""Write tests/golden/planner_goldens.json from the reference's recorded plans.

Reads data files only (JSON results and the cost file) from a reference
checkout; nothing of the reference's code is imported or run.

* results/final/opt/<model>/optimize.json — the profile table the reference
  measured (``profile_table``), the inventory of the per-layer DAG
  (``summary``) and the plan it produced from them (``plan``:
  base_makespan_us, planned_makespan_us, splits).
* configs/planner2_costs.json — the base cost table that plan was laid over.
* results/final/tp_planner/summary.json — the split search on the TP layer
  chain down -> allreduce -> rmsnorm -> qkv, with the per-case inputs of
  scripts/tp_planner.py:15-18 and the allreduce curve of :37-41.
* results/final/planner_robustness/summary.json plus the three valid DAG
  files it checks (dags/e0_tiny_mm_gelu.json, e3_ln_mm.json, e9_mixed.json):
  which graphs the planner accepts and the reason it gives for a reject.

The model configs are the published Qwen shapes; the planner test checks them
against each recorded inventory.

    python tests/golden/make_planner_goldens.py [/root/reference]
"""

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent

CONFIGS = {
    "qwen2.5-0.5b": dict(arch="qwen2.5", hidden_size=896, intermediate_size=4864,
                         num_hidden_layers=24, num_attention_heads=14,
                         num_key_value_heads=2, head_dim=64, vocab_size=151936,
                         qk_norm=False),
    "qwen2.5-7b": dict(arch="qwen2.5", hidden_size=3584, intermediate_size=18944,
                       num_hidden_layers=28, num_attention_heads=28,
                       num_key_value_heads=4, head_dim=128, vocab_size=152064,
                       qk_norm=False),
    "qwen3-vl-4b": dict(arch="qwen3_vl", hidden_size=2560, intermediate_size=9728,
                        num_hidden_layers=36, num_attention_heads=32,
                        num_key_value_heads=8, head_dim=128, vocab_size=151936,
                        qk_norm=True),
    "qwen3-vl-8b": dict(arch="qwen3_vl", hidden_size=4096, intermediate_size=12288,
                        num_hidden_layers=36, num_attention_heads=32,
                        num_key_value_heads=8, head_dim=128, vocab_size=151936,
                        qk_norm=True),
}

# scripts/tp_planner.py:15-18: tag, H, K(down), N(down), down_us,
# allreduce_us, rmsnorm_us, layers; allreduce slope 283 us per tile (:37-41)
TP_CASES = [
    ("qwen2.5-0.5b", 896, 4864, 896, 95.0, 433.9, 30.1, 24),
    ("qwen2.5-7b", 3584, 18944, 3584, 1122.9, 1051.5, 49.0, 28),
]
TP_AR_SLOPE_US = 283.0


def main(ref):
    ref = Path(ref)
    costs = json.loads((ref / "configs/planner2_costs.json").read_text(encoding="utf-8"))
    out = {"base_costs": {k: costs[k] for k in ("launch_us", "traffic_gbps",
                                                 "l2_mb", "event_us", "full")},
           "opt": {}, "tp": {}}
    for model, cfg in CONFIGS.items():
        rec = json.loads((ref / "results/final/opt" / model / "optimize.json")
                         .read_text(encoding="utf-8"))
        out["opt"][model] = {
            "config": cfg,
            "seq": rec["summary"]["seq"],
            "summary": rec["summary"],
            "profile_table": rec["profile_table"],
            "plan": rec["plan"],
        }
    tp = json.loads((ref / "results/final/tp_planner/summary.json").read_text(encoding="utf-8"))
    by_tag = {c["tag"]: c for c in tp["cases"]}
    for tag, H, K, N, down_us, ar_us, rms_us, layers in TP_CASES:
        out["tp"][tag] = {
            "inputs": {"H": H, "K": K, "N": N, "down_us": down_us,
                       "allreduce_us": ar_us, "rmsnorm_us": rms_us,
                       "layers": layers, "allreduce_slope_us": TP_AR_SLOPE_US},
            "expected": by_tag[tag],
        }
    rob = json.loads((ref / "results/final/planner_robustness/summary.json")
                     .read_text(encoding="utf-8"))
    out["robustness"] = {
        "dags": {name: json.loads((ref / "dags" / (name + ".json")).read_text(encoding="utf-8"))
                 for name in ("e0_tiny_mm_gelu", "e3_ln_mm", "e9_mixed")},
        "rows": rob["rows"],
    }
    path = HERE / "planner_goldens.json"
    path.write_text(json.dumps(out, indent=1, ensure_ascii=False) + "\n", encoding="utf-8")
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
