"""Deterministic DAG inputs and the executor checksum, restated in numpy.

Test infrastructure only (see oracle/__init__.py).

* det_values  — DetValue (reference exec/exec_main.cpp:74-79): value i of
  seed s is ((((i*2654435761 + s*40503 + 7) mod 2^32) >> 8) mod 23 - 11)/256.
* node_seed   — FNV-1a(node id) + rank*7919 (exec_main.cpp:491-496).
* input roles — own input seed+1, matmul weight [K,N] seed+2, second operand
  / gamma seed+3 / seed+2 (exec_main.cpp:498-540).
* checksum    — sum over ranks and nodes of the first min(bytes/2, 8192)
  16-bit output words, read in the output's 16-bit format; an fp32 output is
  read as fp16 halves exactly as the reference does (exec_main.cpp:1292-1311).

Pinned by the reference's recorded checksums in results/final/e34_raw.json
(mm->gelu 0.84616 :15, mm->softmax 7.714923 :2301, fan-out 8.846179 :2969),
which the restatement reproduces to < 1e-5 relative
(tests/test_oracle_dag.py).
"""

import numpy as np


def fnv1a(s):
    h = 2166136261
    for c in s.encode():
        h = ((h ^ c) * 16777619) & 0xFFFFFFFF
    return h


def node_seed(node_id, rank):
    return (fnv1a(node_id) + rank * 7919) & 0xFFFFFFFF


def det_values(seed, n, dtype=np.float16):
    """First n DetValue elements for `seed`, as `dtype` (exact in fp16/bf16)."""
    i = np.arange(n, dtype=np.uint64)
    h = (i * np.uint64(2654435761) + np.uint64((seed * 40503) & 0xFFFFFFFF) + np.uint64(7)) \
        & np.uint64(0xFFFFFFFF)
    v = ((h >> np.uint64(8)) % np.uint64(23)).astype(np.int64) - 11
    f = v.astype(np.float32) * np.float32(0.00390625)
    return f.astype(dtype) if dtype is not None else f


def bf16_bits_to_f32(bits):
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def words_as_float(words, out_dtype):
    """16-bit words -> float values as the checksum reads them."""
    if out_dtype == "bf16":
        return bf16_bits_to_f32(words).astype(np.float64)
    return words.view(np.float16).astype(np.float64)


def checksum_words(words, out_dtype):
    return float(words_as_float(np.asarray(words)[:8192], out_dtype).sum())
