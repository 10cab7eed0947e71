// Prefill support kernels around the relay path: token-embedding gather,
// rotate-half RoPE, weight re-layout (transpose) and a word fill.
//
// Replaces the reference's aclnnEmbedding (exec/qwen_main.cpp:646-659) and
// aclnnApplyRotaryPosEmb layout 1 (:567-582).
#include "kr_misc.h"

namespace kr {

namespace {

// out[s, :] = table[ids[s], :]; ids outside [0, vocab) produce a zero row.
__global__ void __launch_bounds__(256) EmbedKernel(const uint16_t *table, const int64_t *ids,
                                                   uint16_t *out, int rows, int cols, int64_t vocab)
{
    const int chunks = cols / 8;
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        const int64_t id = ids[r];
        const bool ok = id >= 0 && id < vocab;
        for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
            U16x8 v;
            if (ok) {
                v = LoadU16x8(table + id * cols + c * 8);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v.v[e] = 0;
            }
            StoreU16x8(out + int64_t(r) * cols + c * 8, v);
        }
    }
}

// In place on x[S, heads, D] (row stride ld): for i < D/2
//   x[i]       <- x[i]*cos[i]       - x[i+D/2]*sin[i]
//   x[i+D/2]   <- x[i+D/2]*cos[i+D/2] + x[i]*sin[i+D/2]
// in fp32 with one rounding; cos/sin rows are positions 0..S-1 of [*, D].
template <int DT>
__global__ void __launch_bounds__(256) RopeKernel(uint16_t *x, int64_t ld, int S, int heads, int D,
                                                  const uint16_t *cos_t, const uint16_t *sin_t)
{
    const int half_chunks = D / 16;  // 8-element chunks in one half
    const int64_t total = int64_t(S) * heads * half_chunks;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += int64_t(gridDim.x) * blockDim.x) {
        const int c = int(t % half_chunks);
        const int64_t sh = t / half_chunks;
        const int h = int(sh % heads);
        const int s = int(sh / heads);
        uint16_t *row = x + int64_t(s) * ld + int64_t(h) * D;
        const int i0 = c * 8;
        const int i1 = i0 + D / 2;
        const U16x8 a = LoadU16x8(row + i0);
        const U16x8 b = LoadU16x8(row + i1);
        const U16x8 ca = LoadU16x8(cos_t + int64_t(s) * D + i0);
        const U16x8 sa = LoadU16x8(sin_t + int64_t(s) * D + i0);
        const U16x8 cb = LoadU16x8(cos_t + int64_t(s) * D + i1);
        const U16x8 sb = LoadU16x8(sin_t + int64_t(s) * D + i1);
        U16x8 oa, ob;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x1 = Elem<DT>::Load(a.v[e]);
            const float x2 = Elem<DT>::Load(b.v[e]);
            oa.v[e] = Elem<DT>::Store(RopeFirst(x1, x2, Elem<DT>::Load(ca.v[e]), Elem<DT>::Load(sa.v[e])));
            ob.v[e] = Elem<DT>::Store(RopeSecond(x2, x1, Elem<DT>::Load(cb.v[e]), Elem<DT>::Load(sb.v[e])));
        }
        StoreU16x8(row + i0, oa);
        StoreU16x8(row + i1, ob);
    }
}

// dst[c, r] = src[r, c] for 16-bit elements, 64x64 tiles through LDS.
__global__ void __launch_bounds__(256) TransposeKernel(const uint16_t *src, uint16_t *dst, int R, int C)
{
    __shared__ uint16_t tile[64][65];
    const int r0 = blockIdx.y * 64;
    const int c0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int r = r0 + i, c = c0 + tx;
        if (r < R && c < C) tile[i][tx] = src[int64_t(r) * C + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int c = c0 + i, r = r0 + tx;
        if (r < R && c < C) dst[int64_t(c) * R + r] = tile[tx][i];
    }
}

__global__ void __launch_bounds__(256) FillKernel(int32_t *p, int64_t n, int32_t v)
{
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * blockDim.x)
        p[i] = v;
}

// n bf16 values of about N(0, std^2) from a counter hash (Irwin-Hall sum of
// four uniforms, scaled to unit variance): stand-in activations with the
// bit activity of real ones.
__device__ __forceinline__ uint32_t Hash32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

__global__ void __launch_bounds__(256) RandBf16Kernel(uint16_t *p, int64_t n, uint32_t seed, float std)
{
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * blockDim.x) {
        uint32_t h = Hash32(uint32_t(i) ^ Hash32(seed ^ uint32_t(i >> 32)));
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h = Hash32(h + 0x9e3779b9u);
            s += float(h >> 8) * (1.0f / 16777216.0f);
        }
        const float v = (s - 2.0f) * 1.7320508f * std;
        uint32_t u = __float_as_uint(v);
        u += 0x7fffu + ((u >> 16) & 1u);
        p[i] = uint16_t(u >> 16);
    }
}

}  // namespace

void RandBf16Launch(void *p, int64_t n, uint32_t seed, float std, hipStream_t stream)
{
    if (n <= 0) return;
    const int grid = int(std::min<int64_t>((n + 255) / 256, 8192));
    hipLaunchKernelGGL(RandBf16Kernel, dim3(grid), dim3(256), 0, stream, static_cast<uint16_t *>(p), n, seed, std);
    Check(hipGetLastError(), "rand fill launch");
}

void EmbedLaunch(const void *table, const int64_t *ids, void *out, int rows, int cols, int64_t vocab,
                 hipStream_t stream)
{
    if (rows <= 0) return;
    if (cols % 8 != 0) throw std::runtime_error("embedding: cols must be a multiple of 8");
    const int grid = rows < 4096 ? rows : 4096;
    hipLaunchKernelGGL(EmbedKernel, dim3(grid), dim3(256), 0, stream, static_cast<const uint16_t *>(table),
                       ids, static_cast<uint16_t *>(out), rows, cols, vocab);
    Check(hipGetLastError(), "embedding launch");
}

void RopeLaunch(int dtype, void *x, int64_t ld, int S, int heads, int D, const void *cos_t,
                const void *sin_t, hipStream_t stream)
{
    if (S <= 0 || heads <= 0) return;
    if (D % 16 != 0) throw std::runtime_error("rope: head_dim must be a multiple of 16");
    const int64_t total = int64_t(S) * heads * (D / 16);
    const int grid = int(std::min<int64_t>((total + 255) / 256, 8192));
    auto *xp = static_cast<uint16_t *>(x);
    auto *cp = static_cast<const uint16_t *>(cos_t);
    auto *sp = static_cast<const uint16_t *>(sin_t);
    if (dtype == kBF16) {
        hipLaunchKernelGGL(RopeKernel<kBF16>, dim3(grid), dim3(256), 0, stream, xp, ld, S, heads, D, cp, sp);
    } else if (dtype == kF16) {
        hipLaunchKernelGGL(RopeKernel<kF16>, dim3(grid), dim3(256), 0, stream, xp, ld, S, heads, D, cp, sp);
    } else {
        throw std::runtime_error("rope: dtype must be bf16 or f16");
    }
    Check(hipGetLastError(), "rope launch");
}

void TransposeLaunch(const void *src, void *dst, int R, int C, hipStream_t stream)
{
    if (R <= 0 || C <= 0) return;
    const dim3 grid((C + 63) / 64, (R + 63) / 64);
    hipLaunchKernelGGL(TransposeKernel, grid, dim3(256), 0, stream, static_cast<const uint16_t *>(src),
                       static_cast<uint16_t *>(dst), R, C);
    Check(hipGetLastError(), "transpose launch");
}

void FillLaunch(int32_t *p, int64_t n, int32_t v, hipStream_t stream)
{
    if (n <= 0) return;
    const int grid = int(std::min<int64_t>((n + 255) / 256, 4096));
    hipLaunchKernelGGL(FillKernel, dim3(grid), dim3(256), 0, stream, p, n, v);
    Check(hipGetLastError(), "fill launch");
}

}  // namespace kr
