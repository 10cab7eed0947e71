// Row arithmetic shared by the standalone row kernel (kr_rowops.hip) and the
// relay consumer that runs inside the producer GEMM (kr_gemm.hip): a row has
// the same bits whichever of them computes it, so a relay split stays
// bit-exact against the serial schedule.
#pragma once

#include "kr_common.h"
#include "kr_relay.h"

namespace kr {

typedef uint32_t RowU32x4 __attribute__((ext_vector_type(4)));

// 16 bytes at byte offset `off` of a wave-uniform base, loaded at device
// scope (sc1: coherent with other XCDs' device-scope stores, without
// invalidating this XCD's L2). The loads are ordinary to the compiler, so
// several stay in flight and the waits are its own.
__device__ __forceinline__ uint4 LoadU128Dev(const void *base, int off)
{
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), short(0), 0x7fffffff, 0x00020000);
    const RowU32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16 /* sc1 */);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Add+RMSNorm of one row of `cols` 16-bit values by one wave: lane ln owns
// the 16-byte chunks ln, ln + 64, ... (CPL of them; cols / 8 <= 64 * CPL).
//   s = bf16(a + b)                      -> sum (optional)
//   rstd = 1 / sqrt(mean(s^2) + eps)     -> rstd_out[0] (optional, fp32)
//   y = bf16(gamma * bf16(s * rstd))
// The sum of squares is accumulated per lane over its chunks in order, then
// over the 64 lanes by the butterfly of WaveSum. Split into load steps and a
// finish step: the loads are branch-free (a lane's chunks past the row end
// re-read its last chunk and are never used), so several rows' loads and
// gamma stay in flight together and the finish step waits only for its own
// row's data, never for earlier rows' stores.
template <int CPL>
struct RowIn {
    uint4 a[CPL];
    uint4 b[CPL];
};

__device__ __forceinline__ int RowChunk(int ln, int c, int chunks) { return min(ln + c * 64, chunks - 1); }

template <int CPL>
__device__ __forceinline__ void RowGammaLoad(const uint16_t *gamma, int cols, int ln, uint4 (&g)[CPL])
{
#pragma unroll
    for (int c = 0; c < CPL; ++c) g[c] = *reinterpret_cast<const uint4 *>(gamma + RowChunk(ln, c, cols / 8) * 8);
}

// B_DEV: b was written by other workgroups of the running kernel (read at
// device scope; b must be wave-uniform).
template <int CPL, bool B_DEV>
__device__ __forceinline__ void AddRmsNormLoad(const uint16_t *a, const uint16_t *b, int cols, int ln, RowIn<CPL> &in)
{
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ch = RowChunk(ln, c, cols / 8);
        in.a[c] = *reinterpret_cast<const uint4 *>(a + ch * 8);
        if constexpr (B_DEV) {
            in.b[c] = LoadU128Dev(b, ch * 16);
        } else {
            in.b[c] = *reinterpret_cast<const uint4 *>(b + ch * 8);
        }
    }
}

// coh: store at device scope (outputs a relay releases).
template <int DT, int CPL>
__device__ __forceinline__ void AddRmsNormFinish(const RowIn<CPL> &in, const uint4 (&g)[CPL], uint16_t *y,
                                                 uint16_t *sum, float *rstd_out, int cols, float eps, int ln, bool coh)
{
    const int chunks = cols / 8;
    float v[CPL][8];
    bool ok[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ch = ln + c * 64;
        ok[c] = ch < chunks;
        if (ok[c]) {
            U16x8 x, w, s;
            *reinterpret_cast<uint4 *>(x.v) = in.a[c];
            *reinterpret_cast<uint4 *>(w.v) = in.b[c];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s.v[e] = Elem<DT>::Store(Elem<DT>::Load(x.v[e]) + Elem<DT>::Load(w.v[e]));
                v[c][e] = Elem<DT>::Load(s.v[e]);
            }
            if (sum != nullptr) PutU128(sum + ch * 8, *reinterpret_cast<const uint4 *>(s.v), coh);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[c][e] = 0.0f;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
    ss = WaveSum(ss);
    const float rstd = 1.0f / sqrtf(ss / float(cols) + eps);
    if (rstd_out != nullptr && ln == 0) PutU32(rstd_out, __float_as_uint(rstd), coh);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        if (!ok[c]) continue;
        U16x8 gv, o;
        *reinterpret_cast<uint4 *>(gv.v) = g[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) o.v[e] = Elem<DT>::Store(Elem<DT>::Load(gv.v[e]) * RoundTo<DT>(v[c][e] * rstd));
        PutU128(y + (ln + c * 64) * 8, *reinterpret_cast<const uint4 *>(o.v), coh);
    }
}

template <int DT, int CPL, bool B_DEV>
__device__ __forceinline__ void AddRmsNormRow(const uint16_t *a, const uint16_t *b, const uint16_t *gamma,
                                              uint16_t *y, uint16_t *sum, float *rstd_out, int cols, float eps,
                                              int ln, bool coh)
{
    uint4 g[CPL];
    RowGammaLoad<CPL>(gamma, cols, ln, g);
    RowIn<CPL> in;
    AddRmsNormLoad<CPL, B_DEV>(a, b, cols, ln, in);
    AddRmsNormFinish<DT, CPL>(in, g, y, sum, rstd_out, cols, eps, ln, coh);
}

// Chunks per lane of a one-wave row of `cols` 16-bit values, as the row
// kernels round it (1, 2, 4 or 8); 0 when the row is not one wave's (the
// standalone kernel then uses 16 or 256 lanes per row).
inline int AddRmsNormRowCpl(int cols)
{
    const int chunks = cols / 8;
    if (cols % 8 != 0 || chunks <= 16 || chunks > 512) return 0;
    const int cpl = (chunks + 63) / 64;
    return cpl <= 1 ? 1 : (cpl <= 2 ? 2 : (cpl <= 4 ? 4 : 8));
}

}  // namespace kr
