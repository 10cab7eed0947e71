// Host interface of the consumer kernels (see kr_rowops.hip).
#pragma once

#include "kr_common.h"
#include "kr_relay.h"

namespace kr {

enum EwOp : int {
    kEwGelu = 0,
    kEwSilu = 1,
    kEwCast = 2,
    kEwMul = 3,
    kEwAdd = 4,
    kEwSwiglu = 5,
    kEwSwigluGU = 6,  // x0 = fused [rows, 2*cols] gate/up, interleaved in groups of 8 columns
};
enum RowOp : int { kRowSoftmax = 0, kRowRmsNorm = 1, kRowAddRmsNorm = 2, kRowLayerNorm = 3 };

// Elementwise op over a [rows, cols] tensor (cols % 8 == 0).
//   gelu/silu/cast : y = f(x0)
//   mul/add        : y = x0 (*|+) x1
//   swiglu         : y = bf16(silu(x0)) * x1   (gate = x0, up = x1)
struct EwDesc {
    int op = kEwGelu;
    int dtype_in = kBF16;
    int dtype_out = kBF16;       // differs from dtype_in only for cast
    const void *x0 = nullptr;
    const void *x1 = nullptr;
    void *y = nullptr;
    int rows = 0, cols = 0;
    int tile_rows = 0;           // relay granularity; 0 = rows (one tile)
    int grid = 0;                // workgroups; 0 = sized to the tensor
    RelayWait wait{};
    RelayPub pub{};
};

// Row-reduction op over [rows, cols] (cols % 8 == 0, cols <= 16384).
//   softmax     : y = softmax(x0) along cols
//   rmsnorm     : y = bf16(gamma * bf16(x0 * rstd)), rstd = 1/sqrt(mean(x0^2)+eps)
//   add_rmsnorm : s = bf16(x0 + x1); y = rmsnorm(s); sum_out = s
//   layernorm   : y = (x0 - mean) / sqrt(var + eps) * gamma + x1 (x1 = the
//                 bias [cols]; biased variance, one rounding)
// rstd_out (fp32 [rows]) and sum_out are optional.
struct RowDesc {
    int op = kRowSoftmax;
    int dtype = kBF16;
    const void *x0 = nullptr;
    const void *x1 = nullptr;
    const void *gamma = nullptr;
    void *y = nullptr;
    void *sum_out = nullptr;
    float *rstd_out = nullptr;
    int rows = 0, cols = 0;
    // Input row r lives at (r / in_group) * in_ld + (r % in_group) * cols
    // (0 = packed rows); outputs are always packed. Lets per-head norms read
    // heads straight out of a fused [S, heads*D + ...] buffer.
    int in_group = 0;
    int64_t in_ld = 0;
    float eps = 1e-6f;
    int tile_rows = 0;
    int grid = 0;
    RelayWait wait{};
    RelayPub pub{};
};

void EwLaunch(const EwDesc &d, hipStream_t stream);
void RowLaunch(const RowDesc &d, hipStream_t stream);

// Several unary consumers of the same rows fused into one pass: every row of
// x is read once and each output written from registers. Each output's bits
// equal its standalone kernel's (same per-element arithmetic; softmax and
// rmsnorm use RowLaunch's lane layout and reduction tree for these cols).
// Ops: kEwGelu, kEwSilu, kEwCast (to `dtype`), kFanSoftmax, kFanRmsNorm
// (gamma). The relay wait is shared; `states` lists every consumer's state
// base (states[0] == wait.state0), all advanced by this launch.
enum FanOp : int { kFanSoftmax = 16, kFanRmsNorm = 17 };
constexpr int kMaxFanOut = 4;
struct FanOutDesc {
    int op = kEwGelu;
    int dtype = kBF16;
    void *y = nullptr;
    const void *gamma = nullptr;
};
struct FanDesc {
    int dtype_in = kBF16;
    const void *x = nullptr;
    int rows = 0, cols = 0;
    float eps = 1e-6f;
    int n_out = 0;
    FanOutDesc out[kMaxFanOut];
    int tile_rows = 0;
    int grid = 0;
    RelayWait wait{};
    int32_t states[kMaxFanOut] = {0, 0, 0, 0};
};
void FanLaunch(const FanDesc &d, hipStream_t stream);

// Standalone relay kernels (the reference's separate kr_wait_* / kr_publish_*
// launches): wait for producer rows [lo, hi) and consume edges adv_lo..adv_hi;
// publish tile `tile` once (arrivals forced to 1).
void WaitLaunch(const RelayWait &w, int lo, int hi, hipStream_t stream);
// The same for a launch standing in for n fused consumers (states[0] ==
// w.state0): every consumer's state blocks adv_lo..adv_hi advance.
void WaitLaunchMulti(const RelayWait &w, int lo, int hi, const int32_t *states, int n, hipStream_t stream);


void PublishLaunch(const RelayPub &p, int tile, hipStream_t stream);

}  // namespace kr
