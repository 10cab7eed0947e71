// Consumer kernels: elementwise and row-reduction ops with the relay
// prologue (wait on the producer tiles that cover a tile's rows) and
// epilogue (release the tile to the next consumer).
//
// Replaces the reference's aclnnGelu / aclnnSoftmax(dim=1) / aclnnCast
// (exec/runtime/op_impl.cpp:214-233), aclnnSilu + aclnnMul
// (exec/qwen_main.cpp:616-644), aclnnAdd (:514-529), aclnnRmsNorm (:531-546)
// and aclnnAddRmsNorm (:548-565).
//
// Work is walked tile by tile (tile = tile_rows rows). Every workgroup waits
// for tile t, processes its share of tile t with a grid stride, arrives on
// tile t's release, then moves on: with a bounded grid the kernel is a
// persistent consumer whose spinning workgroups can never occupy more than
// `grid` slots, so the producer always keeps CUs to make progress.
//
// Arithmetic is in fp32 with one rounding per stored tensor, matching the
// storage rounding of the reference's op sequence. Row reductions use a fixed
// tree (per-lane serial, then xor-butterfly, then waves in index order) that
// depends only on `cols`, never on the tiling, so split == unsplit bit-exact.
#include "kr_rowops.h"
#include "kr_rowcore.h"

#include <algorithm>

namespace kr {

namespace {

constexpr int kThreads = 256;

// ----------------------------------------------------------------- elementwise
struct EwParams {
    const uint16_t *x0;
    const uint16_t *x1;
    void *y;
    int64_t tile_chunks;
    int64_t total_chunks;
    int rows, tile_rows, n_tiles;
    RelayWait w;
    RelayPub pub;
};

template <int OP, int DTI, int DTO>
__global__ void __launch_bounds__(kThreads) EwKernel(EwParams p)
{
    const int64_t stride = int64_t(gridDim.x) * kThreads;
    const bool coh = p.pub.ctrl != nullptr;  // released tiles: device-scope stores
    for (int t = 0; t < p.n_tiles; ++t) {
        const int r_lo = t * p.tile_rows;
        const int r_hi = min(r_lo + p.tile_rows, p.rows);
        RelayWaitRows(p.w, r_lo, r_hi);
        const int64_t c0 = int64_t(t) * p.tile_chunks;
        const int64_t c1 = min(c0 + p.tile_chunks, p.total_chunks);
        if constexpr (DTO == kF32) {
            // 4 values per step (8-byte loads, 16-byte stores): every store
            // instruction of the wave covers whole 128-byte lines of y
            static_assert(OP == kEwCast || OP == kEwGelu || OP == kEwSilu, "fp32 output of a unary op");
            for (int64_t h = 2 * c0 + int64_t(blockIdx.x) * kThreads + threadIdx.x; h < 2 * c1; h += stride) {
                const uint2 u = *reinterpret_cast<const uint2 *>(p.x0 + h * 4);
                const uint16_t a[4] = {uint16_t(u.x), uint16_t(u.x >> 16), uint16_t(u.y), uint16_t(u.y >> 16)};
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = Elem<DTI>::Load(a[e]);
                    o[e] = OP == kEwGelu ? GeluTanh(x) : (OP == kEwSilu ? Silu(x) : x);
                }
                PutU128(static_cast<float *>(p.y) + h * 4,
                        make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                   __float_as_uint(o[3])), coh);
            }
        } else {
            for (int64_t c = c0 + int64_t(blockIdx.x) * kThreads + threadIdx.x; c < c1; c += stride) {
                U16x8 a, b;
                if constexpr (OP == kEwSwigluGU) {
                    // fused gate/up rows: 8 gate columns then the matching 8 up columns
                    a = LoadU16x8(p.x0 + c * 16);
                    b = LoadU16x8(p.x0 + c * 16 + 8);
                } else {
                    a = LoadU16x8(p.x0 + c * 8);
                    if constexpr (OP == kEwMul || OP == kEwAdd || OP == kEwSwiglu) b = LoadU16x8(p.x1 + c * 8);
                }
                float o[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = Elem<DTI>::Load(a.v[e]);
                    if constexpr (OP == kEwGelu) {
                        o[e] = GeluTanh(x);
                    } else if constexpr (OP == kEwSilu) {
                        o[e] = Silu(x);
                    } else if constexpr (OP == kEwCast) {
                        o[e] = x;
                    } else if constexpr (OP == kEwMul) {
                        o[e] = x * Elem<DTI>::Load(b.v[e]);
                    } else if constexpr (OP == kEwAdd) {
                        o[e] = x + Elem<DTI>::Load(b.v[e]);
                    } else {  // swiglu: the silu result is stored (rounded) before the multiply
                        o[e] = RoundTo<DTI>(Silu(x)) * Elem<DTI>::Load(b.v[e]);
                    }
                }
                U16x8 r;
#pragma unroll
                for (int e = 0; e < 8; ++e) r.v[e] = Elem<DTO>::Store(o[e]);
                PutU128(static_cast<uint16_t *>(p.y) + c * 8, *reinterpret_cast<const uint4 *>(r.v), coh);
            }
        }
        RelayArrive(p.pub, t);
    }
    RelayFinish(p.w);
}

// ------------------------------------------------------------------ row ops
struct RowParams {
    const uint16_t *x0;
    const uint16_t *x1;
    const uint16_t *gamma;
    uint16_t *y;
    uint16_t *sum_out;
    float *rstd_out;
    int rows, cols, tile_rows, n_tiles;
    int in_group;
    int64_t in_ld;
    float eps;
    RelayWait w;
    RelayPub pub;
};

// Sum / max over the LPR lanes that own one row. LPR == 256 crosses waves
// through LDS; the caller guarantees the whole workgroup calls it together.
template <int LPR, bool MAX>
__device__ __forceinline__ float GroupReduce(float v, float *red)
{
    if constexpr (LPR <= 64) {
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) {
            const float u = __shfl_xor(v, o, 64);
            v = MAX ? fmaxf(v, u) : v + u;
        }
        return v;
    } else {
        v = MAX ? WaveMax(v) : WaveSum(v);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        if (MAX) return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        return ((red[0] + red[1]) + red[2]) + red[3];
    }
}

template <int OP, int DT, int LPR, int CPL>
__global__ void __launch_bounds__(kThreads) RowKernel(RowParams p)
{
    constexpr int RPB = kThreads / LPR;
    __shared__ float red[4];
    const int slot = threadIdx.x / LPR;
    const int ln = threadIdx.x % LPR;
    const int chunks = p.cols / 8;
    const bool coh = p.pub.ctrl != nullptr;  // released tiles: device-scope stores

    for (int t = 0; t < p.n_tiles; ++t) {
        const int r_lo = t * p.tile_rows;
        const int r_hi = min(r_lo + p.tile_rows, p.rows);
        RelayWaitRows(p.w, r_lo, r_hi);
        for (int rb = r_lo + int(blockIdx.x) * RPB; rb < r_hi; rb += int(gridDim.x) * RPB) {
            const int r = rb + slot;
            const bool active = r < r_hi;
            const int rr = active ? r : r_lo;
            const int64_t base = int64_t(rr) * p.cols;
            const int64_t ibase = int64_t(rr / p.in_group) * p.in_ld + int64_t(rr % p.in_group) * p.cols;
            if constexpr (OP == kRowAddRmsNorm && LPR == 64) {
                // one row per wave: the row code the producer GEMM's relay
                // consumer runs too (kr_rowcore.h), so both give the same bits
                if (active)
                    AddRmsNormRow<DT, CPL, false>(p.x0 + ibase, p.x1 + ibase, p.gamma, p.y + base,
                                                  p.sum_out != nullptr ? p.sum_out + base : nullptr,
                                                  p.rstd_out != nullptr ? p.rstd_out + r : nullptr, p.cols, p.eps, ln,
                                                  coh);
                continue;
            }
            float v[CPL][8];
            bool ok[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int ch = ln + c * LPR;
                ok[c] = active && ch < chunks;
                if (ok[c]) {
                    const U16x8 a = LoadU16x8(p.x0 + ibase + ch * 8);
                    if constexpr (OP == kRowAddRmsNorm) {
                        const U16x8 b = LoadU16x8(p.x1 + ibase + ch * 8);
                        U16x8 s;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            s.v[e] = Elem<DT>::Store(Elem<DT>::Load(a.v[e]) + Elem<DT>::Load(b.v[e]));
                            v[c][e] = Elem<DT>::Load(s.v[e]);
                        }
                        if (p.sum_out != nullptr) PutU128(p.sum_out + base + ch * 8, *reinterpret_cast<const uint4 *>(s.v), coh);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[c][e] = Elem<DT>::Load(a.v[e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[c][e] = 0.0f;
                }
            }

            if constexpr (OP == kRowSoftmax) {
                float m = -INFINITY;
#pragma unroll
                for (int c = 0; c < CPL; ++c)
                    if (ok[c])
#pragma unroll
                        for (int e = 0; e < 8; ++e) m = fmaxf(m, v[c][e]);
                m = GroupReduce<LPR, true>(m, red);
                float s = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c)
                    if (ok[c])
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            v[c][e] = FastExp(v[c][e] - m);
                            s += v[c][e];
                        }
                s = GroupReduce<LPR, false>(s, red);
                // one IEEE division per row; every element scales by it
                const float inv = 1.0f / s;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    if (!ok[c]) continue;
                    U16x8 o;
#pragma unroll
                    for (int e = 0; e < 8; ++e) o.v[e] = Elem<DT>::Store(v[c][e] * inv);
                    PutU128(p.y + base + (ln + c * LPR) * 8, *reinterpret_cast<const uint4 *>(o.v), coh);
                }
            } else if constexpr (OP == kRowLayerNorm) {
                // mean, then the biased variance about it (two passes over
                // the registers), then one rounding of the affine result
                float s1 = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c)
#pragma unroll
                    for (int e = 0; e < 8; ++e) s1 += v[c][e];
                const float mean = GroupReduce<LPR, false>(s1, red) / float(p.cols);
                float s2 = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c)
                    if (ok[c])
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const float d = v[c][e] - mean;
                            s2 += d * d;
                        }
                const float rstd = 1.0f / sqrtf(GroupReduce<LPR, false>(s2, red) / float(p.cols) + p.eps);
                if (p.rstd_out != nullptr && active && ln == 0) PutU32(p.rstd_out + r, __float_as_uint(rstd), coh);
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    if (!ok[c]) continue;
                    const int ch = ln + c * LPR;
                    const U16x8 g = LoadU16x8(p.gamma + ch * 8), bb = LoadU16x8(p.x1 + ch * 8);
                    U16x8 o;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        o.v[e] = Elem<DT>::Store((v[c][e] - mean) * rstd * Elem<DT>::Load(g.v[e]) + Elem<DT>::Load(bb.v[e]));
                    PutU128(p.y + base + ch * 8, *reinterpret_cast<const uint4 *>(o.v), coh);
                }
            } else {
                float ss = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c)
#pragma unroll
                    for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
                ss = GroupReduce<LPR, false>(ss, red);
                const float rstd = 1.0f / sqrtf(ss / float(p.cols) + p.eps);
                if (p.rstd_out != nullptr && active && ln == 0) PutU32(p.rstd_out + r, __float_as_uint(rstd), coh);
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    if (!ok[c]) continue;
                    const int ch = ln + c * LPR;
                    const U16x8 g = LoadU16x8(p.gamma + ch * 8);
                    U16x8 o;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        o.v[e] = Elem<DT>::Store(Elem<DT>::Load(g.v[e]) * RoundTo<DT>(v[c][e] * rstd));
                    PutU128(p.y + base + ch * 8, *reinterpret_cast<const uint4 *>(o.v), coh);
                }
            }
        }
        RelayArrive(p.pub, t);
    }
    RelayFinish(p.w);
}

// ------------------------------------------------- fused sibling consumers
struct FanOutParams {
    int op, dtype;
    void *y;
    const uint16_t *gamma;
};
struct FanParams {
    const uint16_t *x;
    int rows, cols, tile_rows, n_tiles;
    float eps;
    int n_out;
    FanOutParams out[kMaxFanOut];
    RelayWait w;
    int32_t states[kMaxFanOut];
};

typedef uint32_t FanU32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void FanPut16(uint16_t *p, const U16x8 &r)
{
    __builtin_nontemporal_store(*reinterpret_cast<const FanU32x4 *>(r.v), reinterpret_cast<FanU32x4 *>(p));
}

// Store eight fp32 values of one 16-byte input chunk as output type DTO.
__device__ __forceinline__ void FanStore(void *y, int64_t elem, int dto, const float (&o)[8])
{
    if (dto == kF32) {
        FanU32x4 *yp = reinterpret_cast<FanU32x4 *>(static_cast<float *>(y) + elem);
        const FanU32x4 lo = {__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])};
        const FanU32x4 hi = {__float_as_uint(o[4]), __float_as_uint(o[5]), __float_as_uint(o[6]), __float_as_uint(o[7])};
        __builtin_nontemporal_store(lo, yp);
        __builtin_nontemporal_store(hi, yp + 1);
        return;
    }
    U16x8 r;
    if (dto == kBF16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) r.v[e] = Elem<kBF16>::Store(o[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) r.v[e] = Elem<kF16>::Store(o[e]);
    }
    FanPut16(static_cast<uint16_t *>(y) + elem, r);
}

// The row loop, lane layout (LPR lanes per row, CPL chunks per lane) and
// reduction tree of RowKernel, with every output computed from the one load.
// At most 128 registers per wave: the kernel spins on the CUs of the GEMM
// that produces its rows (136 registers per wave for the co-resident tiles),
// and a CU must hold one workgroup of each; at full width four waves per SIMD
// keep a 1024-workgroup grid resident in one round.
// Rows are read once and outputs written once: non-temporal accesses, so the
// consumer does not evict the operand lines the GEMM beside it reuses.
template <int DT, int LPR, int CPL>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) FanKernel(FanParams p)
{
    constexpr int RPB = kThreads / LPR;
    __shared__ float red[4];
    const int slot = threadIdx.x / LPR;
    const int ln = threadIdx.x % LPR;
    const int chunks = p.cols / 8;

    for (int t = 0; t < p.n_tiles; ++t) {
        const int r_lo = t * p.tile_rows;
        const int r_hi = min(r_lo + p.tile_rows, p.rows);
        RelayWaitRows(p.w, r_lo, r_hi);
        for (int rb = r_lo + int(blockIdx.x) * RPB; rb < r_hi; rb += int(gridDim.x) * RPB) {
            const int r = rb + slot;
            const bool active = r < r_hi;
            const int64_t base = int64_t(active ? r : r_lo) * p.cols;
            float v[CPL][8];
            bool ok[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int ch = ln + c * LPR;
                ok[c] = active && ch < chunks;
                if (ok[c]) {
                    U16x8 a;
                    *reinterpret_cast<FanU32x4 *>(a.v) =
                        __builtin_nontemporal_load(reinterpret_cast<const FanU32x4 *>(p.x + base + ch * 8));
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[c][e] = Elem<DT>::Load(a.v[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[c][e] = 0.0f;
                }
            }
            for (int i = 0; i < p.n_out; ++i) {
                const FanOutParams &o = p.out[i];
                if (o.op == kFanSoftmax) {
                    // the last output (FanLaunch orders it so): exponentials
                    // replace the row in registers, as in RowKernel
                    float m = -INFINITY;
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
                        if (ok[c])
#pragma unroll
                            for (int e = 0; e < 8; ++e) m = fmaxf(m, v[c][e]);
                    m = GroupReduce<LPR, true>(m, red);
                    float s = 0.0f;
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
                        if (ok[c])
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                v[c][e] = FastExp(v[c][e] - m);
                                s += v[c][e];
                            }
                    s = GroupReduce<LPR, false>(s, red);
                    const float inv = 1.0f / s;
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        if (!ok[c]) continue;
                        U16x8 q;
#pragma unroll
                        for (int e = 0; e < 8; ++e) q.v[e] = Elem<DT>::Store(v[c][e] * inv);
                        FanPut16(static_cast<uint16_t *>(o.y) + base + (ln + c * LPR) * 8, q);
                    }
                } else if (o.op == kFanRmsNorm) {
                    float ss = 0.0f;
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
#pragma unroll
                        for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
                    ss = GroupReduce<LPR, false>(ss, red);
                    const float rstd = 1.0f / sqrtf(ss / float(p.cols) + p.eps);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        if (!ok[c]) continue;
                        const int ch = ln + c * LPR;
                        const U16x8 g = LoadU16x8(o.gamma + ch * 8);
                        U16x8 q;
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            q.v[e] = Elem<DT>::Store(Elem<DT>::Load(g.v[e]) * RoundTo<DT>(v[c][e] * rstd));
                        FanPut16(static_cast<uint16_t *>(o.y) + base + ch * 8, q);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        if (!ok[c]) continue;
                        float q[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            q[e] = o.op == kEwGelu ? GeluTanh(v[c][e]) : (o.op == kEwSilu ? Silu(v[c][e]) : v[c][e]);
                        FanStore(o.y, base + (ln + c * LPR) * 8, o.dtype, q);
                    }
                }
            }
        }
    }
    RelayFinishMulti(p.w, p.states, p.n_out);
}

__global__ void __launch_bounds__(64) WaitKernel(RelayWait w, int lo, int hi)
{
    RelayWaitRows(w, lo, hi);
    RelayFinish(w);
}

struct WaitStates {
    int32_t s[kMaxFanOut];
    int n;
};

// Wait for rows [lo, hi), then consume the edges of every listed consumer
// (fused sibling consumers share one wait).
__global__ void __launch_bounds__(64) WaitMultiKernel(RelayWait w, int lo, int hi, WaitStates st)
{
    RelayWaitRows(w, lo, hi);
    RelayFinishMulti(w, st.s, st.n);
}

__global__ void __launch_bounds__(64) PublishKernel(RelayPub p, int tile) { RelayArrive(p, tile); }

int TileCount(int rows, int tile_rows) { return (rows + tile_rows - 1) / tile_rows; }

template <int OP>
void EwDispatch(const EwDesc &d, const EwParams &p, int grid, hipStream_t s)
{
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, s, p); };
    if (OP == kEwCast) {
        if (d.dtype_in == kBF16 && d.dtype_out == kF16) return go(EwKernel<kEwCast, kBF16, kF16>);
        if (d.dtype_in == kBF16 && d.dtype_out == kF32) return go(EwKernel<kEwCast, kBF16, kF32>);
        if (d.dtype_in == kF16 && d.dtype_out == kF32) return go(EwKernel<kEwCast, kF16, kF32>);
        if (d.dtype_in == kF16 && d.dtype_out == kBF16) return go(EwKernel<kEwCast, kF16, kBF16>);
        throw std::runtime_error("cast: unsupported dtype pair");
    }
    if (d.dtype_in != d.dtype_out) throw std::runtime_error("elementwise: dtype_in != dtype_out");
    if (d.dtype_in == kBF16) return go(EwKernel<OP, kBF16, kBF16>);
    if (d.dtype_in == kF16) return go(EwKernel<OP, kF16, kF16>);
    throw std::runtime_error("elementwise: dtype must be bf16 or f16");
}

template <int OP, int DT>
void RowDispatchT(const RowParams &p, int lpr, int cpl, int grid, hipStream_t s)
{
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, s, p); };
    if (lpr == 16) return go(RowKernel<OP, DT, 16, 1>);
    if (lpr == 64) {
        switch (cpl) {
            case 1: return go(RowKernel<OP, DT, 64, 1>);
            case 2: return go(RowKernel<OP, DT, 64, 2>);
            case 4: return go(RowKernel<OP, DT, 64, 4>);
            default: return go(RowKernel<OP, DT, 64, 8>);
        }
    }
    switch (cpl) {
        case 1: return go(RowKernel<OP, DT, 256, 1>);
        case 2: return go(RowKernel<OP, DT, 256, 2>);
        case 4: return go(RowKernel<OP, DT, 256, 4>);
        default: return go(RowKernel<OP, DT, 256, 8>);
    }
}

template <int OP>
void RowDispatch(const RowDesc &d, const RowParams &p, int lpr, int cpl, int grid, hipStream_t s)
{
    if (d.dtype == kBF16) return RowDispatchT<OP, kBF16>(p, lpr, cpl, grid, s);
    if (d.dtype == kF16) return RowDispatchT<OP, kF16>(p, lpr, cpl, grid, s);
    throw std::runtime_error("row op: dtype must be bf16 or f16");
}

void CheckAligned(const void *p, const char *what)
{
    if (reinterpret_cast<uintptr_t>(p) & 15) throw std::runtime_error(std::string(what) + " must be 16-byte aligned");
}

// Lanes per row for a row of `chunks` 16-byte chunks: up to 4096 16-bit
// columns one wave owns a row (up to 8 chunks per lane, all in flight at
// once; reductions stay inside the wave), wider rows take the whole
// workgroup. The layout fixes the reduction tree, so every kernel that
// reduces rows of a given width uses this one choice.
int RowLanes(int chunks) { return chunks <= 16 ? 16 : (chunks <= 512 ? 64 : 256); }

}  // namespace

void EwLaunch(const EwDesc &d, hipStream_t stream)
{
    if (d.rows <= 0 || d.cols <= 0) return;
    if (d.cols % 8 != 0) throw std::runtime_error("elementwise: cols must be a multiple of 8");
    CheckAligned(d.x0, "elementwise x0");
    CheckAligned(d.y, "elementwise y");
    const bool binary = d.op == kEwMul || d.op == kEwAdd || d.op == kEwSwiglu;
    if (binary) CheckAligned(d.x1, "elementwise x1");
    EwParams p{};
    p.x0 = static_cast<const uint16_t *>(d.x0);
    p.x1 = static_cast<const uint16_t *>(d.x1);
    p.y = d.y;
    p.rows = d.rows;
    p.tile_rows = d.tile_rows > 0 ? d.tile_rows : d.rows;
    p.n_tiles = TileCount(d.rows, p.tile_rows);
    p.tile_chunks = int64_t(p.tile_rows) * d.cols / 8;
    p.total_chunks = int64_t(d.rows) * d.cols / 8;
    p.w = d.wait;
    p.pub = d.pub;
    int grid = d.grid;
    if (grid <= 0) {
        const int64_t want = (p.tile_chunks + kThreads - 1) / kThreads;
        grid = int(std::min<int64_t>(std::max<int64_t>(want, 1), 4096));
    }
    p.pub.arrivals = grid;
    switch (d.op) {
        case kEwGelu: return EwDispatch<kEwGelu>(d, p, grid, stream);
        case kEwSilu: return EwDispatch<kEwSilu>(d, p, grid, stream);
        case kEwCast: return EwDispatch<kEwCast>(d, p, grid, stream);
        case kEwMul: return EwDispatch<kEwMul>(d, p, grid, stream);
        case kEwAdd: return EwDispatch<kEwAdd>(d, p, grid, stream);
        case kEwSwiglu: return EwDispatch<kEwSwiglu>(d, p, grid, stream);
        case kEwSwigluGU: return EwDispatch<kEwSwigluGU>(d, p, grid, stream);
        default: throw std::runtime_error("elementwise: unknown op");
    }
}

void RowLaunch(const RowDesc &d, hipStream_t stream)
{
    if (d.rows <= 0 || d.cols <= 0) return;
    if (d.cols % 8 != 0) throw std::runtime_error("row op: cols must be a multiple of 8");
    if (d.cols > 16384) throw std::runtime_error("row op: cols must be <= 16384");
    CheckAligned(d.x0, "row op x0");
    CheckAligned(d.y, "row op y");
    if (d.op == kRowAddRmsNorm) CheckAligned(d.x1, "add_rmsnorm x1");
    if (d.op == kRowLayerNorm) CheckAligned(d.x1, "layernorm bias");
    if (d.op != kRowSoftmax) CheckAligned(d.gamma, "rmsnorm gamma");
    if (d.sum_out) CheckAligned(d.sum_out, "add_rmsnorm sum");
    RowParams p{};
    p.x0 = static_cast<const uint16_t *>(d.x0);
    p.x1 = static_cast<const uint16_t *>(d.x1);
    p.gamma = static_cast<const uint16_t *>(d.gamma);
    p.y = static_cast<uint16_t *>(d.y);
    p.sum_out = static_cast<uint16_t *>(d.sum_out);
    p.rstd_out = d.rstd_out;
    p.rows = d.rows;
    p.cols = d.cols;
    p.in_group = d.in_group > 0 ? d.in_group : 1;
    p.in_ld = d.in_ld > 0 ? d.in_ld : int64_t(d.cols) * p.in_group;
    if (p.in_ld % 8 != 0) throw std::runtime_error("row op: in_ld must be a multiple of 8");
    p.eps = d.eps;
    p.tile_rows = d.tile_rows > 0 ? d.tile_rows : d.rows;
    p.n_tiles = TileCount(d.rows, p.tile_rows);
    p.w = d.wait;
    p.pub = d.pub;
    const int chunks = d.cols / 8;
    const int lpr = RowLanes(chunks);
    int cpl = (chunks + lpr - 1) / lpr;
    cpl = cpl <= 1 ? 1 : (cpl <= 2 ? 2 : (cpl <= 4 ? 4 : 8));
    const int rpb = kThreads / lpr;
    int grid = d.grid;
    if (grid <= 0) grid = std::max(1, std::min((p.tile_rows + rpb - 1) / rpb, 8192));
    p.pub.arrivals = grid;
    switch (d.op) {
        case kRowSoftmax: return RowDispatch<kRowSoftmax>(d, p, lpr, cpl, grid, stream);
        case kRowRmsNorm: return RowDispatch<kRowRmsNorm>(d, p, lpr, cpl, grid, stream);
        case kRowAddRmsNorm: return RowDispatch<kRowAddRmsNorm>(d, p, lpr, cpl, grid, stream);
        case kRowLayerNorm: return RowDispatch<kRowLayerNorm>(d, p, lpr, cpl, grid, stream);
        default: throw std::runtime_error("row op: unknown op");
    }
}

namespace {

template <int DT>
void FanDispatch(const FanParams &p, int lpr, int cpl, int grid, hipStream_t s)
{
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, s, p); };
    if (lpr == 16) return go(FanKernel<DT, 16, 1>);
    if (lpr == 64) {
        switch (cpl) {
            case 1: return go(FanKernel<DT, 64, 1>);
            case 2: return go(FanKernel<DT, 64, 2>);
            case 4: return go(FanKernel<DT, 64, 4>);
            default: return go(FanKernel<DT, 64, 8>);
        }
    }
    switch (cpl) {
        case 1: return go(FanKernel<DT, 256, 1>);
        case 2: return go(FanKernel<DT, 256, 2>);
        case 4: return go(FanKernel<DT, 256, 4>);
        default: return go(FanKernel<DT, 256, 8>);
    }
}

}  // namespace

void FanLaunch(const FanDesc &d, hipStream_t stream)
{
    if (d.rows <= 0 || d.cols <= 0) return;
    if (d.n_out < 1 || d.n_out > kMaxFanOut) throw std::runtime_error("fan-out: 1..4 outputs");
    if (d.cols % 8 != 0) throw std::runtime_error("fan-out: cols must be a multiple of 8");
    if (d.cols > 16384) throw std::runtime_error("fan-out: cols must be <= 16384");
    if (d.dtype_in != kBF16 && d.dtype_in != kF16) throw std::runtime_error("fan-out: input must be bf16 or f16");
    CheckAligned(d.x, "fan-out x");
    FanParams p{};
    p.x = static_cast<const uint16_t *>(d.x);
    p.rows = d.rows;
    p.cols = d.cols;
    p.eps = d.eps;
    p.n_out = d.n_out;
    // outputs in kernel order: softmax (which overwrites the row in
    // registers) last; the order of independent outputs changes no bits
    int order[kMaxFanOut], n_soft = 0, j = 0;
    for (int i = 0; i < d.n_out; ++i)
        if (d.out[i].op != kFanSoftmax) order[j++] = i;
    for (int i = 0; i < d.n_out; ++i)
        if (d.out[i].op == kFanSoftmax) {
            order[j++] = i;
            ++n_soft;
        }
    if (n_soft > 1) throw std::runtime_error("fan-out: at most one softmax output");
    for (int i = 0; i < d.n_out; ++i) p.states[i] = d.states[i];
    for (int jj = 0; jj < d.n_out; ++jj) {
        const int i = order[jj];
        const FanOutDesc &o = d.out[i];
        CheckAligned(o.y, "fan-out y");
        const bool ew = o.op == kEwGelu || o.op == kEwSilu || o.op == kEwCast;
        if (!ew && o.op != kFanSoftmax && o.op != kFanRmsNorm) throw std::runtime_error("fan-out: unsupported op");
        if (o.op != kEwCast && o.dtype != d.dtype_in) throw std::runtime_error("fan-out: only cast changes dtype");
        if (o.op == kFanRmsNorm) CheckAligned(o.gamma, "fan-out gamma");
        p.out[jj] = {o.op, o.dtype, o.y, static_cast<const uint16_t *>(o.gamma)};
    }
    if (d.wait.ctrl != nullptr && d.states[0] != d.wait.state0)
        throw std::runtime_error("fan-out: states[0] must be the wait's state block");
    p.tile_rows = d.tile_rows > 0 ? d.tile_rows : d.rows;
    p.n_tiles = TileCount(d.rows, p.tile_rows);
    p.w = d.wait;
    const int chunks = d.cols / 8;
    const int lpr = RowLanes(chunks);
    int cpl = (chunks + lpr - 1) / lpr;
    cpl = cpl <= 1 ? 1 : (cpl <= 2 ? 2 : (cpl <= 4 ? 4 : 8));
    const int rpb = kThreads / lpr;
    int grid = d.grid;
    if (grid <= 0) grid = std::max(1, std::min((p.tile_rows + rpb - 1) / rpb, 8192));
    if (d.dtype_in == kBF16) FanDispatch<kBF16>(p, lpr, cpl, grid, stream);
    else FanDispatch<kF16>(p, lpr, cpl, grid, stream);
    Check(hipGetLastError(), "fan-out launch");
}

void WaitLaunchMulti(const RelayWait &w, int lo, int hi, const int32_t *states, int n, hipStream_t stream)
{
    if (w.ctrl == nullptr) return;
    if (n < 1 || n > kMaxFanOut) throw std::runtime_error("wait: 1..4 consumer states");
    if (states[0] != w.state0) throw std::runtime_error("wait: states[0] must be the wait's state block");
    WaitStates st{};
    for (int i = 0; i < n; ++i) st.s[i] = states[i];
    st.n = n;
    hipLaunchKernelGGL(WaitMultiKernel, dim3(1), dim3(64), 0, stream, w, lo, hi, st);
    Check(hipGetLastError(), "wait launch");
}

void WaitLaunch(const RelayWait &w, int lo, int hi, hipStream_t stream)
{
    if (w.ctrl == nullptr) return;
    hipLaunchKernelGGL(WaitKernel, dim3(1), dim3(64), 0, stream, w, lo, hi);
    Check(hipGetLastError(), "wait launch");
}

void PublishLaunch(const RelayPub &p, int tile, hipStream_t stream)
{
    if (p.ctrl == nullptr) return;
    RelayPub q = p;
    q.arrivals = 1;
    hipLaunchKernelGGL(PublishKernel, dim3(1), dim3(64), 0, stream, q, tile);
    Check(hipGetLastError(), "publish launch");
}

}  // namespace kr
