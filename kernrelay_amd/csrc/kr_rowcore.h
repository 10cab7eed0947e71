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
// over the 64 lanes by the butterfly of WaveSum. B_DEV: b was written by
// other workgroups of the running kernel (read at device scope). coh: store
// at device scope (outputs a relay releases).
template <int DT, int CPL, bool B_DEV>
__device__ __forceinline__ void AddRmsNormRow(const uint16_t *a, const uint16_t *b, const uint16_t *gamma,
                                              uint16_t *y, uint16_t *sum, float *rstd_out, int cols, float eps,
                                              int ln, bool coh)
{
    const int chunks = cols / 8;
    float v[CPL][8];
    bool ok[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ch = ln + c * 64;
        ok[c] = ch < chunks;
        if (ok[c]) {
            const U16x8 x = LoadU16x8(a + ch * 8);
            U16x8 w;
            if constexpr (B_DEV) {
                *reinterpret_cast<uint4 *>(w.v) = LoadU128Dev(b, ch * 16);
            } else {
                w = LoadU16x8(b + ch * 8);
            }
            U16x8 s;
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
        const int ch = ln + c * 64;
        const U16x8 g = LoadU16x8(gamma + ch * 8);
        U16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o.v[e] = Elem<DT>::Store(Elem<DT>::Load(g.v[e]) * RoundTo<DT>(v[c][e] * rstd));
        PutU128(y + ch * 8, *reinterpret_cast<const uint4 *>(o.v), coh);
    }
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
