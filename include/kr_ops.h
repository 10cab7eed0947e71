/*
 * KernRelay-MI355X op-level C ABI (exported by libkernrelay.so).
 *
 * These are the hand-written HIP kernels behind the runtimes, callable on
 * caller-owned device memory. Each replaces one closed CANN aclnn call site
 * of the reference (cited per function). All calls are asynchronous on
 * `stream` (a hipStream_t, NULL = default stream), return 0 on success and a
 * non-zero code on invalid arguments or launch failure; kr_ops_last_error()
 * then describes the failure (thread-local, valid until the next call).
 *
 * Tensors are row-major; 16-bit element types are passed as raw bits.
 * Pointers to 16-bit tensors must be 16-byte aligned and row lengths
 * multiples of 8 elements (the kernels move 16-byte vectors).
 */
#ifndef KR_OPS_H
#define KR_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
enum { KR_BF16 = 0, KR_F16 = 1, KR_F32 = 2 };

/* Elementwise ops for kr_op_elementwise. */
enum {
    KR_EW_GELU = 0,
    KR_EW_SILU = 1,
    KR_EW_CAST = 2,
    KR_EW_MUL = 3,
    KR_EW_ADD = 4,
    KR_EW_SWIGLU = 5,     /* y = bf16(silu(x0)) * x1 */
    KR_EW_SWIGLU_GU = 6   /* x0 = fused [rows, 2*cols] gate/up in 8-column groups */
};

/* Row-reduction ops for kr_op_rowop. */
enum {
    KR_ROW_SOFTMAX = 0,
    KR_ROW_RMSNORM = 1,
    KR_ROW_ADD_RMSNORM = 2,
    KR_ROW_LAYERNORM = 3  /* gamma = weight [cols], x1 = bias [cols] (aclnnLayerNorm,
                             reference exec/runtime/op_impl.cpp:237-254) */
};

/* Relay control blocks: 8 x int32 each, zero-initialised once by the owner
 * (layout: published, consumed, status, arrive, done, timed_out, -, -; the
 * first three words are the reference's kernels/kr_sync_common.h:10-15). */
#define KR_CTRL_WORDS 8

/* Consumer side: wait for the producer tiles that cover the rows a launch
 * reads. Local row r is producer row r + row_off; producer tile k covers
 * rows [k*prod_rows, (k+1)*prod_rows), its flag is block flag0 + k and the
 * consumer's state for it is block state0 + k; state blocks adv_lo..adv_hi-1
 * are consumed by this launch. ctrl == NULL disables waiting.
 * Replaces reference kernels/kr_wait_aiv.cpp:7-36 (kr_wait_aiv/aic). */
typedef struct kr_wait {
    int32_t *ctrl;
    int32_t flag0;
    int32_t state0;
    int32_t prod_rows;
    int32_t row_off;
    int32_t adv_lo;
    int32_t adv_hi;
    uint32_t max_spins; /* 0 = default bound */
} kr_wait;

/* Producer side: tile t (rows [t*rows_per_tile, (t+1)*rows_per_tile) of the
 * launch) releases flag block flag0 + t when its last workgroup finishes.
 * `arrivals` is filled in by the library. ctrl == NULL disables publishing.
 * Replaces reference kernels/kr_publish_aiv.cpp:6-23 (kr_publish_aiv/aic). */
typedef struct kr_pub {
    int32_t *ctrl;
    int32_t flag0;
    int32_t rows_per_tile;
    int32_t arrivals;
} kr_pub;

const char *kr_ops_last_error(void);

/* C[M,N] = A[M,K] . Bt[N,K]^T (+ bias[N], rounded as matmul-then-add);
 * bf16/f16 in and out, fp32 accumulate. bm = M tile (0 = automatic; 64,
 * 128 or 256). pub may be NULL. wait may be NULL; else every workgroup waits
 * for the producer tiles covering its rows of A before loading them (the
 * GEMM as a relay consumer), and the launch consumes wait->adv_lo..adv_hi.
 * Replaces aclnnMatmul (reference exec/qwen_main.cpp:499-512,
 * exec/runtime/op_impl.cpp:175-201) and the fused QKV bias Add (:1336-1344);
 * the wait replaces a kr_wait_aic launch ahead of it (qwen_main.cpp:672-688). */
int kr_op_gemm(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C,
               int64_t ldc, const void *bias, int M, int N, int K, int bm, const kr_wait *wait,
               const kr_pub *pub, void *stream);

/* Gate/up GEMM with its SwiGLU consumer in the same launch: C[M, 2*cols] =
 * A[M,K] . Bt[2*cols,K]^T (gate/up interleaved in groups of 8 columns) is
 * released in row tiles through pub (required; rows_per_tile divides M), and
 * workgroups appended after the GEMM's own wait for each released tile and
 * write act[M, cols] = SwiGLU over its rows (silu rounded to 16 bits before
 * the multiply, as kr_op_elementwise's swiglu_gu). Appended workgroups are
 * dispatched after every GEMM workgroup, so they only take CUs the GEMM's
 * last round leaves idle. tail_tiles (0 = all) limits the appended consumer
 * to the first relay tiles (the caller runs SwiGLU on the rest); order_rows
 * (0 = the relay tile) sets the row runs in which the GEMM produces. Replaces the relay edge matmul_gate/up ->
 * Silu -> Mul of the reference (exec/qwen_main.cpp:616-644, 888-889). */
int kr_op_gemm_swiglu(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C,
                      void *act, int M, int cols, int K, const kr_pub *pub, int tail_tiles,
                      int order_rows, void *stream);

/* Gate/up GEMM with SwiGLU applied in its epilogue (the relay of
 * matmul_gate/up -> Silu -> Mul at MFMA-tile granularity, handed over in
 * registers): for A[M,K] . Bt[2*cols,K]^T with gate/up interleaved in groups
 * of 8 columns, writes act[M, cols] (row stride ld_act) =
 * bf16(bf16(silu(gate)) * up) with the rounding of kr_op_elementwise's
 * swiglu_gu over the stored product; the [M, 2*cols] product itself is not
 * written. cols must be a multiple of 8. Replaces the same reference call
 * sites as kr_op_gemm_swiglu (exec/qwen_main.cpp:616-644, 888-889). */
int kr_op_gemm_swiglu_epilogue(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *act,
                               int64_t ld_act, int M, int cols, int K, void *stream);

/* Row-tiled relay of a projection to its Add+RMSNorm consumer (the
 * reference's down -> Add+RMSNorm tile loop, exec/qwen_main.cpp:1274-1302,
 * on one device and without the all-reduce; the consumer is aclnnAddRmsNorm,
 * :548-565): C[M,N] = A . Bt^T is released in relay tiles of
 * pub->rows_per_tile rows through pub's control blocks, and as soon as a
 * tile is released the launch's own workgroups compute, for each of its rows,
 * sum = bf16(res + C) and y = bf16(gamma * bf16(sum * rstd)),
 * rstd = 1/sqrt(mean(sum^2) + eps) (rstd_out fp32 [M], optional; sum may be
 * NULL), bit-identical to kr_op_rowop(KR_ROW_ADD_RMSNORM) over C. Each
 * release is consumed by the same launch: the tile's block ends with
 * consumed advanced and status 1 (2 if a wait ran past max_spins). C, res,
 * y and sum are packed [M, N]; N in 136..4096, a multiple of 8. ws/counters
 * as for kr_op_gemm_streamk (NULL: data-parallel tiles). Fails (non-zero)
 * when a relay tile's producer workgroups cannot all be resident at once:
 * use smaller relay tiles. */
int kr_op_gemm_add_rmsnorm(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C, int M,
                           int N, int K, const void *res, const void *gamma, void *y, void *sum, float *rstd_out,
                           float eps, const kr_pub *pub, uint32_t max_spins, void *ws, size_t ws_bytes,
                           int32_t *counters, int n_counters, void *stream);

/* Stream-K GEMM for shapes whose 256x256 output tiles are fewer than the CUs
 * (the reference's q/k/v, o and down projections at prefill sizes,
 * exec/qwen_main.cpp:499-512, 1336-1344): every CU takes an equal run of the
 * (tile, K stage) iterations, and a tile split between CUs is summed in fixed
 * piece order by the last of them, so the bits depend on the shape only (a
 * row-split launch of the same GEMM would differ; use it where no launch is
 * split). Same operands and rounding as kr_op_gemm (bias added to the
 * stored product). ws/counters: caller-owned device memory of at least the
 * sizes kr_op_gemm_streamk_workspace reports; the counters must be zero
 * before the first launch and are left zero; launches sharing them must be
 * ordered (one stream). A shape the plan does not cover (0 bytes reported)
 * runs as kr_op_gemm. */
int kr_op_gemm_streamk_workspace(int M, int N, int K, size_t *ws_bytes, int *counters);
int kr_op_gemm_streamk(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C, int64_t ldc,
                       const void *bias, int M, int N, int K, void *ws, size_t ws_bytes, int32_t *counters,
                       int n_counters, void *stream);

/* kr_op_gemm_streamk without a workspace argument, allocating nothing: the
 * partial sums and tile counters live in a device array of the library
 * (48 MiB of partials, 1024 counters; each GPU it runs on holds one until
 * the process ends). No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc). Same plan, piece order and bits as
 * kr_op_gemm_streamk; the counters are cleared at every call. Shapes whose
 * split needs more than the array holds fail with an error naming both
 * sizes. All calls on one GPU share the array: calls that may overlap in
 * time on one GPU (different streams, or host threads without ordering)
 * race and must not be issued. */
int kr_op_gemm_streamk_noalloc(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C,
                               int64_t ldc, const void *bias, int M, int N, int K, void *stream);

/* Elementwise op on [rows, cols]; x1 used by mul/add/swiglu; dtype_out
 * differs from dtype_in only for cast. tile_rows = relay granularity
 * (0 = rows); grid = workgroups (0 = sized to the tensor). wait/pub may be
 * NULL. Replaces aclnnGelu / aclnnCast (reference
 * exec/runtime/op_impl.cpp:214-228), aclnnSilu / aclnnMul / aclnnAdd
 * (exec/qwen_main.cpp:514-529, 616-644). */
int kr_op_elementwise(int op, int dtype_in, int dtype_out, const void *x0, const void *x1, void *y,
                      int rows, int cols, int tile_rows, int grid, const kr_wait *wait,
                      const kr_pub *pub, void *stream);

/* Row op on [rows, cols]: softmax along cols; rmsnorm; add_rmsnorm (x1 =
 * second addend, sum_out = rounded sum). rstd_out (fp32 [rows]) and sum_out
 * may be NULL. Replaces aclnnSoftmax dim=1 (reference
 * exec/runtime/op_impl.cpp:229-233), aclnnRmsNorm and aclnnAddRmsNorm
 * (exec/qwen_main.cpp:531-565). */
int kr_op_rowop(int op, int dtype, const void *x0, const void *x1, const void *gamma, void *y,
                void *sum_out, float *rstd_out, int rows, int cols, float eps, int tile_rows,
                int grid, const kr_wait *wait, const kr_pub *pub, void *stream);

/* Standalone one-workgroup wait for producer rows [lo, hi) (the reference's
 * separate kr_wait_* launch) and standalone release of tile `tile` (the
 * reference's kr_publish_* launch). */
int kr_op_wait(const kr_wait *wait, int lo, int hi, void *stream);
int kr_op_publish(const kr_pub *pub, int tile, void *stream);

/* out[r,:] = table[ids[r],:] (ids int64; out-of-range ids give zero rows).
 * Replaces aclnnEmbedding (reference exec/qwen_main.cpp:646-659). */
int kr_op_embedding(const void *table, const int64_t *ids, void *out, int rows, int cols,
                    int64_t vocab, void *stream);

/* In-place rotate-half RoPE on x[S, heads, D] (row stride ld elements) with
 * cos/sin tables [>=S, D]. Replaces aclnnApplyRotaryPosEmb layout 1
 * (reference exec/qwen_main.cpp:567-582). */
int kr_op_rope(int dtype, void *x, int64_t ld, int S, int heads, int D, const void *cos_t,
               const void *sin_t, void *stream);

/* Causal GQA attention, q [S,HQ,D], k/v [S,HKV,D], out [S,HQ,D], D in {64,128};
 * ld* = row strides in elements (0 = packed heads*D).
 * Replaces aclnnFlashAttentionScore (reference exec/qwen_main.cpp:591-614). */
int kr_op_attention(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk,
                    const void *v, int64_t ldv, void *out, int64_t ldo, int S, int HQ, int HKV,
                    int D, float scale, void *stream);

/* kr_op_attention with long causal rows split across workgroups: query
 * blocks of more than 16 key blocks are cut into up to 4 pieces whose fp32
 * partials the last piece sums in piece order (deterministic; the bits
 * depend on S only). ws / counters of the sizes kr_op_attention_workspace
 * reports (0 bytes: nothing to split, the call runs unsplit); counters zero
 * before the first call and left zero by every call; calls sharing them must
 * not overlap. Same role as kr_op_attention (reference
 * exec/qwen_main.cpp:591-614, FlashN); the split is a scheduling choice of
 * this library with no reference counterpart. */
int kr_op_attention_workspace(int S, int HQ, int D, size_t *ws_bytes, int *counters);
int kr_op_attention_split(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk,
                          const void *v, int64_t ldv, void *out, int64_t ldo, int S, int HQ, int HKV,
                          int D, float scale, void *ws, size_t ws_bytes, int32_t *counters,
                          int n_counters, void *stream);

/* dst[C,R] = src[R,C]^T for 16-bit elements (weight re-layout at load; the
 * reference stores matmul weights as weight_t [K,N], scripts/export_model.py:159-161). */
int kr_op_transpose(const void *src, void *dst, int R, int C, void *stream);

/* A stream with a hardware queue of its own (CU-masked to every CU). Two
 * relay parties that wait on each other on the device must not share a queue
 * (a queue runs its kernels in order); ordinary streams are multiplexed onto
 * a few queues. Returns NULL on failure. No reference counterpart: the
 * reference's two streams feed separate AIC and AIV engines
 * (exec/qwen_main.cpp:206-209). */
void *kr_op_stream_create(void);
int kr_op_stream_destroy(void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KR_OPS_H */
