// Host interface of the producer GEMM (see kr_gemm.hip).
#pragma once

#include "kr_common.h"
#include "kr_relay.h"

namespace kr {

struct GemmDesc {
    int dtype = kBF16;           // kBF16 or kF16 (inputs and output)
    const void *A = nullptr;     // [M, K], row stride lda (elements)
    const void *Bt = nullptr;    // [N, K], row stride ldb (weights, K contiguous)
    void *C = nullptr;           // [M, N], row stride ldc
    const void *bias = nullptr;  // optional [N]
    int64_t lda = 0, ldb = 0, ldc = 0;
    int M = 0, N = 0, K = 0;
    int bm = 0;                  // M tile (0 = pick automatically)
    int bn = 0;                  // N tile (0 = pick automatically)
    RelayPub pub{};              // pub.ctrl == nullptr: no release
    RelayWait wait{};            // wait.ctrl == nullptr: A is ready; else each
                                 // workgroup waits for the tiles of A it reads
    // Tail consumer (requires pub; C = interleaved gate/up, ldc = 2*tail_cols):
    // workgroups appended to the grid wait for each released relay tile and
    // write SwiGLU of its rows into tail_act [M, tail_cols].
    void *tail_act = nullptr;
    int tail_cols = 0;
    int tail_tiles = 0;          // relay tiles the tail consumes (0 = all); the
                                 // rest are left to a kernel after the GEMM
    bool coresident = false;     // a consumer kernel spins on the same CUs while
                                 // this GEMM runs: use a tile whose workgroup
                                 // leaves register room beside it (not 256x256)
    // SwiGLU epilogue (the in-register relay of gate/up to its consumer):
    // C's columns are gate/up interleaved in groups of 8; instead of C the
    // launch writes epi_act[M, N/2] (row stride ld_act) = bf16(silu(gate))*up,
    // rounded as the standalone SwiGLU kernel rounds. C is not written.
    void *epi_act = nullptr;
    int64_t ld_act = 0;
    // Unary consumer written beside C (the in-register relay of a GEMM to a
    // GELU / SiLU / cast consumer): y[M, N] (row stride ld_y, dtype y_dtype)
    // = f(C) for KR_EW_GELU, KR_EW_SILU or KR_EW_CAST, computed from each
    // stored 16-bit C value exactly as the elementwise kernel computes it.
    void *y = nullptr;
    int y_op = 0;
    int y_dtype = 0;
    int64_t ld_y = 0;
    // Stream-K (no relay on this launch): when the 256x256 tiles are fewer
    // than the CUs, every CU takes an equal share of the (tile, K stage)
    // iterations and split tiles are summed in piece order by their last
    // piece. Needs the caller's workspace (GemmStreamKNeeds); the counters
    // must be zero before the first launch and stay owned by one stream.
    // Bits depend on the shape only, so a launch that never runs row-split
    // is reproducible; silently data-parallel when the plan does not apply.
    bool streamk = false;
    void *sk_ws = nullptr;
    size_t sk_ws_bytes = 0;
    int32_t *sk_cnt = nullptr;
    int sk_cnt_len = 0;
    // RoPE epilogue: columns [0, rope_cols) of C are heads of rope_d (64 or
    // 128) values rotated after the bias, as the standalone RoPE kernel
    // rotates the stored product (row r at position rope_pos0 + r; tables
    // [positions, rope_d]). rope_cols % rope_d == 0.
    const void *rope_cos = nullptr;
    const void *rope_sin = nullptr;
    int rope_cols = 0;
    int rope_d = 0;
    int rope_pos0 = 0;
    int order_rows = 0;          // > 0: produce in runs of this many rows (a
                                 // multiple of pub.rows_per_tile), default
                                 // one run per relay tile
    // Add+RMSNorm relay consumer (requires pub; C packed, ldc == N; N a
    // one-wave row, 136..4096 columns): once a relay tile is released, the
    // producer's own workgroups compute, for each of its rows,
    //   norm_sum = res + C,  norm_y = rmsnorm(norm_sum) * gamma
    // ([M, N] packed; norm_rstd fp32 [M] optional) with the standalone
    // Add+RMSNorm kernel's row code (same bits). The edge's control blocks
    // are pub's: each relay tile's release is consumed by this launch
    // (consumed + 1, status 1 = ok, 2 = a wait exceeded norm_max_spins).
    // Only where every relay tile's producer workgroups fit the device at
    // once (GemmLaunch throws otherwise).
    const void *norm_res = nullptr;
    const void *norm_gamma = nullptr;
    void *norm_y = nullptr;
    void *norm_sum = nullptr;
    float *norm_rstd = nullptr;
    float norm_eps = 1e-6f;
    uint32_t norm_max_spins = kDefaultMaxSpins;
};

// Launch C = A . Bt^T (+bias). pub.rows_per_tile (when publishing) must be a
// multiple of the chosen M tile; pub.arrivals is computed here.
// With tail_act, workgroups appended after the GEMM's own consume its tiles:
// workgroups are dispatched in id order, so they only take CUs the GEMM's
// last round leaves idle, and each starts on a relay tile once released. With a wait,
// every workgroup first waits for the producer tiles covering its rows of A,
// and the launch consumes wait.adv_lo..adv_hi once all workgroups are done.
void GemmLaunch(const GemmDesc &d, hipStream_t stream);

// True when GemmLaunch can run the Add+RMSNorm relay consumer for this shape
// and relay tile (rows_per_tile): a one-wave row width, whole tiles, and the
// producer workgroups of one relay tile resident at once (device slots from
// the occupancy of the kernel instantiation the launch runs).
bool GemmNormRelayFits(int M, int N, int K, int rows_per_tile, bool streamk_ws, int dtype = kBF16);

// Workspace a stream-K launch of this shape needs (0 bytes, 0 counters: the
// launch runs data-parallel).
void GemmStreamKNeeds(int M, int N, int K, size_t *ws_bytes, int *counters);

struct GemmTile {
    int bm, bn;
};

// Tile the launcher would use for this shape ({-1,-1} when no M tile divides
// the relay tile). coresident: skip 256x256, whose four waves take every
// register of the CU (a workgroup of a concurrently spinning consumer would
// otherwise keep the CU from the GEMM).
GemmTile GemmPickTile(int M, int N, int relay_rows, bool coresident = false);

}  // namespace kr
