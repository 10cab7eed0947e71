/*
 * KernRelay-MI355X stable C ABI (the drop-in boundary).
 *
 * Same six symbols, argument meaning, ownership and error convention as the
 * reference's include/kernrelay.h:11-69, so an existing ctypes caller
 * (reference python/kernrelay/libapi.py:20-132) binds this library unchanged.
 *
 * Ownership: every `const char*` argument is borrowed for the duration of the
 * call. `out`/`out_cap` is a caller-owned buffer that receives NUL-terminated
 * JSON; when `out_cap` is smaller than the JSON plus its terminator the call
 * fails with {"error":"output buffer too small"} (reference
 * exec/qwen_main.cpp:2302-2312).
 *
 * Threading: one call at a time per process (the reference documents the
 * entry points as process-level, include/kernrelay.h:22-24). On HIP repeated
 * calls in one process are safe; concurrent calls are not supported.
 */
#ifndef KERNRELAY_H
#define KERNRELAY_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version string; static storage, caller does not free.
 * Replaces reference exec/kr_api.cpp:9-12. */
const char *kr_version(void);

/*
 * Run one KernRelay schedule.json (the nhp_exec equivalent) on one GPU.
 *   schedule_json : schedule produced by kernrelay_amd.schedule
 *                   (build_fixed_schedule / serial_schedule)
 *   iters/warmup  : timed and untimed executions
 *   devices       : "0" or "0,0" (one entry per rank; every rank runs on the
 *                   listed device); NULL/"" = device 0 for every rank
 *   mode          : "direct" | "graph" | "graph_per_stream" | "graph_segment"
 *                   (graph_segment: one graph per run of a lane between
 *                   cross-lane waits, the segments joined by events)
 *   out_json      : path that receives the result JSON
 * Returns 0 on success; 2 for NULL arguments or usage errors; 1 on any other
 * failure (message on stderr).
 * Replaces reference exec/kr_api.cpp:23-46 -> exec/exec_main.cpp:1325-1494.
 */
int kr_plan_run(const char *schedule_json, int iters, int warmup,
                const char *devices, const char *mode, const char *out_json);

/*
 * Single-GPU Qwen2.5 / Qwen3-text prefill from a model directory
 * (manifest.json + weights.bin + ids.bin [+ ref_last_logits.bin, ref.json]).
 * mode: serial | serial_fused | serial_graph | graph_whole |
 *       relay_event | relay_flag | relay_flag_graph |
 *       relay_split | relay_split:<k> | relay_split:<k>:<edges>
 *         (row-tiled relay, k in 1..8, default 4; graph-replayed; edges =
 *          o+down | o | down | none names the flag edges o -> Add+RMSNorm
 *          and down -> Add+RMSNorm; default: every edge whose relay tiles
 *          fit the device; the gate/up GEMM always hands SwiGLU its tiles
 *          in its epilogue)
 * Result JSON keys follow reference exec/qwen_main.cpp:1785-1803.
 * Returns 0 on success; 1 with {"error":...} in `out` on failure.
 * Replaces reference exec/qwen_main.cpp:2287-2314.
 */
int kr_qwen_run(const char *model_dir, const char *mode, int seq, int device,
                int warmup, int iters, char *out, size_t out_cap);

/*
 * Two-GPU pipeline-parallel prefill. Not built on this single-GPU target:
 * always returns 1 with {"error":"multi-GPU not in scope"}.
 * Replaces reference exec/qwen_main.cpp:2256-2285.
 */
int kr_qwen_pp_run(const char *model_dir, const char *mode, int seq, int dev0,
                   int dev1, int requests, int warmup, int iters, char *out,
                   size_t out_cap);

/*
 * Two-GPU tensor-parallel MLP prefill. Not built on this single-GPU target:
 * always returns 1 with {"error":"multi-GPU not in scope"}.
 * Replaces reference exec/qwen_main.cpp:2225-2254.
 */
int kr_qwen_tp_run(const char *model_dir, const char *mode, int seq, int dev0,
                   int dev1, int tiles, int warmup, int iters, char *out,
                   size_t out_cap);

/*
 * Per-op k-tile cost table: spec_json names a file holding
 * {"cases":[{"op":"matmul_gate","k":1}, ...]}; every case runs k row slices
 * of the op captured into one hipGraph and replayed (reference
 * exec/qwen_main.cpp:1535-1783). Ops: matmul_q/k/v/o/gate/up/down/lm, add,
 * rmsnorm, add_rmsnorm, rope, silu, mul, swiglu, embedding, attention.
 * Returns 0 on success; 1 with {"error":...} in `out` on failure.
 * Replaces reference exec/qwen_main.cpp:2198-2223.
 */
int kr_qwen_profile_many(const char *model_dir, const char *spec_json, int seq,
                         int device, char *out, size_t out_cap);

#ifdef __cplusplus
}
#endif

#endif /* KERNRELAY_H */
