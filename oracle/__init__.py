"""CPU oracle for the KernRelay relay path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only to check results (or as the timed CPU baseline),
never as the thing measured or shipped. The product (kernrelay_amd/ and
libkernrelay.so) never imports it.

Modules
  dag_inputs  the reference's deterministic DAG inputs and checksum
              (exec/exec_main.cpp:74-79, 491-540, 1292-1311), numpy
  ops         fp32 torch-CPU restatement of every op on the path, each stored
              tensor rounded to its 16-bit storage type
  qwen        Qwen2.5 / Qwen3-text prefill in the reference's op order
              (exec/qwen_main.cpp:925-992) over a model directory
  dag_eval    node outputs of a schedule.json's DAG (first rows or full)
  relay_model a CPU thread model of the device flag protocol
  hf_reference transformers' Qwen2/Qwen3ForCausalLM on a model directory:
              the independent writer of ref_last_logits.bin / ref.json and
              the pin of qwen's composition

How each function is pinned (golden vectors, closed forms, brute force,
library routines) is listed in each module header; tests/test_oracle_*.py
hold the checks.
"""
