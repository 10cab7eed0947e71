// C ABI of the op-level kernels (include/kr_ops.h).
#include "../../include/kr_ops.h"

#include <mutex>
#include <string>
#include <vector>

#include <hip/hip_ext.h>

#include "kr_gemm.h"
#include "kr_misc.h"
#include "kr_rowops.h"

static_assert(sizeof(kr_wait) == sizeof(kr::RelayWait), "kr_wait layout");
static_assert(offsetof(kr_wait, max_spins) == offsetof(kr::RelayWait, max_spins), "kr_wait layout");
static_assert(sizeof(kr_pub) == sizeof(kr::RelayPub), "kr_pub layout");
static_assert(offsetof(kr_pub, arrivals) == offsetof(kr::RelayPub, arrivals), "kr_pub layout");

namespace {

thread_local std::string g_last_error;

template <typename F>
int Guard(F &&f)
{
    try {
        g_last_error.clear();
        f();
        return 0;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return 1;
    }
}

kr::RelayWait ToWait(const kr_wait *w)
{
    kr::RelayWait r{};
    if (w == nullptr || w->ctrl == nullptr) return r;
    r.ctrl = w->ctrl;
    r.flag0 = w->flag0;
    r.state0 = w->state0;
    r.prod_rows = w->prod_rows;
    r.row_off = w->row_off;
    r.adv_lo = w->adv_lo;
    r.adv_hi = w->adv_hi;
    r.max_spins = w->max_spins ? w->max_spins : kr::kDefaultMaxSpins;
    if (r.prod_rows <= 0) throw std::runtime_error("wait: prod_rows must be > 0");
    if (r.row_off < 0) throw std::runtime_error("wait: row_off must be >= 0");
    return r;
}

kr::RelayPub ToPub(const kr_pub *p)
{
    kr::RelayPub r{};
    if (p == nullptr || p->ctrl == nullptr) return r;
    r.ctrl = p->ctrl;
    r.flag0 = p->flag0;
    r.rows_per_tile = p->rows_per_tile;
    if (r.rows_per_tile <= 0) throw std::runtime_error("pub: rows_per_tile must be > 0");
    return r;
}

hipStream_t S(void *s) { return static_cast<hipStream_t>(s); }

// ------------------------------------------------ allocation-free stream-K
// kr_op_gemm_streamk_noalloc keeps the stream-K partial sums and tile
// counters in this file-scope device array instead of a caller workspace:
// 48 MiB of fp32 partials (a split of up to 48 pieces of 256x256 tiles, e.g.
// the Qwen2.5-0.5B down projection 2048x896x4864: 32 MiB) and 1024 tile
// counters. Every GPU the library runs on holds its own copy until the
// process ends. In host code `scratch` names a host-side stand-in, never the
// device memory: its device address comes from hipGetSymbolAddress, once per
// device with that device current, and only that address reaches kernels.
constexpr size_t kScratchPartialBytes = size_t(48) << 20;
constexpr int kScratchCounters = 1024;
static __device__ __align__(256) unsigned char scratch[kScratchPartialBytes + kScratchCounters * 4];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};

// Device address of this device's scratch array (set up on the first call
// on the device, with the device current).
unsigned char *ScratchOnCurrentDevice()
{
    int dev = 0;
    kr::Check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("noalloc: device id out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        kr::Check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_scratch[dev] = p;
    }
    return static_cast<unsigned char *>(g_scratch[dev]);
}

// The counters start every call at zero (a fill kernel, not a memset, so the
// call also works under graph capture).
__global__ void ZeroCountersKernel(int32_t *c, int n)
{
    const int i = int(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) c[i] = 0;
}

}  // namespace

extern "C" {

const char *kr_ops_last_error(void) { return g_last_error.c_str(); }

int kr_op_gemm(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C, int64_t ldc,
               const void *bias, int M, int N, int K, int bm, const kr_wait *wait, const kr_pub *pub, void *stream)
{
    return Guard([&] {
        kr::GemmDesc d;
        d.dtype = dtype;
        d.A = A;
        d.Bt = Bt;
        d.C = C;
        d.bias = bias;
        d.lda = lda;
        d.ldb = ldb;
        d.ldc = ldc;
        d.M = M;
        d.N = N;
        d.K = K;
        d.bm = bm;
        d.pub = ToPub(pub);
        d.wait = ToWait(wait);
        if (d.pub.ctrl && M % d.pub.rows_per_tile != 0) throw std::runtime_error("gemm: M must be a multiple of rows_per_tile");
        kr::GemmLaunch(d, S(stream));
    });
}

int kr_op_gemm_swiglu(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C, void *act, int M,
                      int cols, int K, const kr_pub *pub, int tail_tiles, int order_rows, void *stream)
{
    return Guard([&] {
        kr::GemmDesc d;
        d.dtype = dtype;
        d.A = A;
        d.Bt = Bt;
        d.C = C;
        d.lda = lda;
        d.ldb = ldb;
        d.ldc = 2 * int64_t(cols);
        d.M = M;
        d.N = 2 * cols;
        d.K = K;
        d.pub = ToPub(pub);
        d.tail_act = act;
        d.tail_cols = cols;
        d.tail_tiles = tail_tiles;
        d.order_rows = order_rows;
        kr::GemmLaunch(d, S(stream));
    });
}

int kr_op_gemm_add_rmsnorm(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C, int M,
                           int N, int K, const void *res, const void *gamma, void *y, void *sum, float *rstd_out,
                           float eps, const kr_pub *pub, uint32_t max_spins, void *ws, size_t ws_bytes,
                           int32_t *counters, int n_counters, void *stream)
{
    return Guard([&] {
        if (pub == nullptr || pub->ctrl == nullptr) throw std::runtime_error("gemm add_rmsnorm: needs a relay release");
        kr::GemmDesc d;
        d.dtype = dtype;
        d.A = A;
        d.Bt = Bt;
        d.C = C;
        d.lda = lda;
        d.ldb = ldb;
        d.ldc = N;
        d.M = M;
        d.N = N;
        d.K = K;
        d.pub = ToPub(pub);
        d.norm_res = res;
        d.norm_gamma = gamma;
        d.norm_y = y;
        d.norm_sum = sum;
        d.norm_rstd = rstd_out;
        d.norm_eps = eps;
        d.norm_max_spins = max_spins;
        if (ws != nullptr) {
            d.streamk = true;
            d.sk_ws = ws;
            d.sk_ws_bytes = ws_bytes;
            d.sk_cnt = counters;
            d.sk_cnt_len = n_counters;
        }
        kr::GemmLaunch(d, S(stream));
    });
}

int kr_op_gemm_streamk_workspace(int M, int N, int K, size_t *ws_bytes, int *counters)
{
    return Guard([&] {
        if (ws_bytes == nullptr || counters == nullptr) throw std::runtime_error("null output pointer");
        kr::GemmStreamKNeeds(M, N, K, ws_bytes, counters);
    });
}

int kr_op_gemm_streamk(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C, int64_t ldc,
                       const void *bias, int M, int N, int K, void *ws, size_t ws_bytes, int32_t *counters,
                       int n_counters, void *stream)
{
    return Guard([&] {
        kr::GemmDesc d;
        d.dtype = dtype;
        d.A = A;
        d.Bt = Bt;
        d.C = C;
        d.bias = bias;
        d.lda = lda;
        d.ldb = ldb;
        d.ldc = ldc;
        d.M = M;
        d.N = N;
        d.K = K;
        d.streamk = true;
        d.sk_ws = ws;
        d.sk_ws_bytes = ws_bytes;
        d.sk_cnt = counters;
        d.sk_cnt_len = n_counters;
        kr::GemmLaunch(d, S(stream));
    });
}

int kr_op_gemm_streamk_noalloc(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *C,
                               int64_t ldc, const void *bias, int M, int N, int K, void *stream)
{
    return Guard([&] {
        size_t ws_bytes = 0;
        int counters = 0;
        kr::GemmStreamKNeeds(M, N, K, &ws_bytes, &counters);
        if (ws_bytes > kScratchPartialBytes || counters > kScratchCounters)
            throw std::runtime_error("gemm_streamk_noalloc: this shape's split needs " + std::to_string(ws_bytes) +
                                     " bytes of partials and " + std::to_string(counters) +
                                     " counters; the library's scratch holds " +
                                     std::to_string(kScratchPartialBytes) + " bytes and " +
                                     std::to_string(kScratchCounters) + " counters (use kr_op_gemm_streamk)");
        kr::GemmDesc d;
        d.dtype = dtype;
        d.A = A;
        d.Bt = Bt;
        d.C = C;
        d.bias = bias;
        d.lda = lda;
        d.ldb = ldb;
        d.ldc = ldc;
        d.M = M;
        d.N = N;
        d.K = K;
        if (ws_bytes > 0) {
            unsigned char *base = ScratchOnCurrentDevice();
            int32_t *cnt = reinterpret_cast<int32_t *>(base + kScratchPartialBytes);
            hipLaunchKernelGGL(ZeroCountersKernel, dim3((counters + 255) / 256), dim3(256), 0, S(stream), cnt,
                               counters);
            kr::Check(hipGetLastError(), "zero counters launch");
            d.streamk = true;
            d.sk_ws = base;
            d.sk_ws_bytes = kScratchPartialBytes;
            d.sk_cnt = cnt;
            d.sk_cnt_len = kScratchCounters;
        }
        kr::GemmLaunch(d, S(stream));
    });
}

int kr_op_gemm_swiglu_epilogue(int dtype, const void *A, int64_t lda, const void *Bt, int64_t ldb, void *act,
                               int64_t ld_act, int M, int cols, int K, void *stream)
{
    return Guard([&] {
        kr::GemmDesc d;
        d.dtype = dtype;
        d.A = A;
        d.Bt = Bt;
        d.C = nullptr;
        d.lda = lda;
        d.ldb = ldb;
        d.ldc = 2 * int64_t(cols);
        d.M = M;
        d.N = 2 * cols;
        d.K = K;
        d.epi_act = act;
        d.ld_act = ld_act;
        kr::GemmLaunch(d, S(stream));
    });
}

int kr_op_elementwise(int op, int dtype_in, int dtype_out, const void *x0, const void *x1, void *y, int rows,
                      int cols, int tile_rows, int grid, const kr_wait *wait, const kr_pub *pub, void *stream)
{
    return Guard([&] {
        kr::EwDesc d;
        d.op = op;
        d.dtype_in = dtype_in;
        d.dtype_out = dtype_out;
        d.x0 = x0;
        d.x1 = x1;
        d.y = y;
        d.rows = rows;
        d.cols = cols;
        d.tile_rows = tile_rows;
        d.grid = grid;
        d.wait = ToWait(wait);
        d.pub = ToPub(pub);
        kr::EwLaunch(d, S(stream));
        kr::Check(hipGetLastError(), "elementwise launch");
    });
}

int kr_op_rowop(int op, int dtype, const void *x0, const void *x1, const void *gamma, void *y, void *sum_out,
                float *rstd_out, int rows, int cols, float eps, int tile_rows, int grid, const kr_wait *wait,
                const kr_pub *pub, void *stream)
{
    return Guard([&] {
        kr::RowDesc d;
        d.op = op;
        d.dtype = dtype;
        d.x0 = x0;
        d.x1 = x1;
        d.gamma = gamma;
        d.y = y;
        d.sum_out = sum_out;
        d.rstd_out = rstd_out;
        d.rows = rows;
        d.cols = cols;
        d.eps = eps;
        d.tile_rows = tile_rows;
        d.grid = grid;
        d.wait = ToWait(wait);
        d.pub = ToPub(pub);
        kr::RowLaunch(d, S(stream));
        kr::Check(hipGetLastError(), "row op launch");
    });
}

int kr_op_wait(const kr_wait *wait, int lo, int hi, void *stream)
{
    return Guard([&] { kr::WaitLaunch(ToWait(wait), lo, hi, S(stream)); });
}

int kr_op_publish(const kr_pub *pub, int tile, void *stream)
{
    return Guard([&] {
        kr::RelayPub p = ToPub(pub);
        if (p.ctrl && pub->rows_per_tile <= 0) throw std::runtime_error("publish: bad tile");
        kr::PublishLaunch(p, tile, S(stream));
    });
}

int kr_op_embedding(const void *table, const int64_t *ids, void *out, int rows, int cols, int64_t vocab,
                    void *stream)
{
    return Guard([&] { kr::EmbedLaunch(table, ids, out, rows, cols, vocab, S(stream)); });
}

int kr_op_rope(int dtype, void *x, int64_t ld, int S_, int heads, int D, const void *cos_t, const void *sin_t,
               void *stream)
{
    return Guard([&] { kr::RopeLaunch(dtype, x, ld, S_, heads, D, cos_t, sin_t, S(stream)); });
}

int kr_op_attention(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                    void *out, int64_t ldo, int S_, int HQ, int HKV, int D, float scale, void *stream)
{
    return Guard([&] { kr::AttnLaunch(dtype, q, ldq, k, ldk, v, ldv, out, ldo, S_, HQ, HKV, D, scale, S(stream)); });
}

int kr_op_attention_workspace(int S_, int HQ, int D, size_t *ws_bytes, int *counters)
{
    if (ws_bytes == nullptr || counters == nullptr) return 2;
    return Guard([&] { kr::AttnSplitNeeds(S_, HQ, D, ws_bytes, counters); });
}

int kr_op_attention_split(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v,
                          int64_t ldv, void *out, int64_t ldo, int S_, int HQ, int HKV, int D, float scale, void *ws,
                          size_t ws_bytes, int32_t *counters, int n_counters, void *stream)
{
    return Guard([&] {
        kr::AttnSplit sp;
        sp.ws = static_cast<float *>(ws);
        sp.ws_bytes = ws_bytes;
        sp.cnt = counters;
        sp.cnt_len = n_counters;
        kr::AttnLaunch(dtype, q, ldq, k, ldk, v, ldv, out, ldo, S_, HQ, HKV, D, scale, S(stream), &sp);
    });
}

int kr_op_transpose(const void *src, void *dst, int R, int C, void *stream)
{
    return Guard([&] { kr::TransposeLaunch(src, dst, R, C, S(stream)); });
}

void *kr_op_stream_create(void)
{
    hipStream_t st = nullptr;
    const int rc = Guard([&] {
        int dev = 0;
        kr::Check(hipGetDevice(&dev), "hipGetDevice");
        hipDeviceProp_t prop;
        kr::Check(hipGetDeviceProperties(&prop, dev), "device props");
        std::vector<uint32_t> all((prop.multiProcessorCount + 31) / 32, 0u);
        for (int c = 0; c < prop.multiProcessorCount; ++c) all[c / 32] |= 1u << (c % 32);
        kr::Check(hipExtStreamCreateWithCUMask(&st, uint32_t(all.size()), all.data()), "create stream");
    });
    return rc == 0 ? static_cast<void *>(st) : nullptr;
}

int kr_op_stream_destroy(void *stream)
{
    return Guard([&] { kr::Check(hipStreamDestroy(static_cast<hipStream_t>(stream)), "destroy stream"); });
}

}  // extern "C"
