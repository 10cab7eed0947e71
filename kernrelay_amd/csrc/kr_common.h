// Shared definitions for the KernRelay-MI355X kernels and runtimes.
// gfx950 (CDNA4) only: 64-lane wavefronts, MFMA, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace kr {

// Element type codes shared with the C ABI (include/kr_ops.h).
enum DType : int { kBF16 = 0, kF16 = 1, kF32 = 2 };

inline size_t DTypeBytes(int dt) { return dt == kF32 ? 4 : 2; }

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void Check(hipError_t r, const char *what)
{
    if (r != hipSuccess) {
        throw HipError(std::string(what) + ": " + hipGetErrorString(r));
    }
}

// ---------------------------------------------------------------- host conv
// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
inline uint16_t HostF32ToBF16(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

inline float HostBF16ToF32(uint16_t b)
{
    uint32_t u = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// IEEE half bits -> float (host side, exact).
inline float HostF16ToF32(uint16_t h)
{
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            u = sign | uint32_t(127 - 15 - e) << 23 | (man & 0x3ffu) << 13;
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | man << 13;
    } else {
        u = sign | (exp + 127 - 15) << 23 | man << 13;
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// float -> IEEE half bits, round-to-nearest-even (host side).
inline uint16_t HostF32ToF16(float f)
{
    _Float16 h = static_cast<_Float16>(f);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

// --------------------------------------------------------------- device conv
// 16-bit storage types are moved around as raw bits (uint16_t) and converted
// explicitly, so the rounding of every store is visible in the source.
__device__ __forceinline__ float BF16ToF32(uint16_t b)
{
    return __uint_as_float(uint32_t(b) << 16);
}

// gfx950 v_cvt_pk_bf16_f32: round to nearest even, one instruction (the same
// bits as HostF32ToBF16 for every non-NaN input).
__device__ __forceinline__ uint16_t F32ToBF16(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Workgroup id -> logical work index, XCD-aware. The dispatcher deals
// workgroups to the 8 XCDs round-robin (XCD = blockIdx % 8), each with its
// own L2. Within the run of `per` consecutive ids from `first`, the ids an
// XCD receives map to one contiguous chunk of [0, per), so neighbouring work
// items (sharing operands) run under one L2. A bijection on [0, per).
__device__ __forceinline__ int XcdChunk(int bid, int first, int per)
{
    const int off = (bid - first) & 7;
    const int slot = (bid - first) >> 3;
    const int q = per >> 3, rem = per & 7;
    return off < rem ? off * (q + 1) + slot : rem * (q + 1) + (off - rem) * q + slot;
}

// Fast transcendental building blocks on the hardware's v_exp_f32 (2^x) and
// v_rcp_f32 (about 1 ulp each): far below the 16-bit rounding that follows
// every use, and the same instructions in every schedule (split or not).
__device__ __forceinline__ float FastExp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float FastRcp(float x) { return __builtin_amdgcn_rcpf(x); }

// RoPE (rotate_half layout) of the pair (x1 in the first half of a head, x2
// at the same offset in the second half), with cos / sin at the output
// element's own position: first half x1*c - x2*s, second half x2*c + x1*s.
// Explicit fmas, so the standalone kernel and the GEMM epilogue round alike.
__device__ __forceinline__ float RopeFirst(float x1, float x2, float c, float s) { return __builtin_fmaf(x1, c, -(x2 * s)); }
__device__ __forceinline__ float RopeSecond(float x2, float x1, float c, float s) { return __builtin_fmaf(x2, c, x1 * s); }

// SiLU as every kernel here computes it (x * sigmoid(x)).
__device__ __forceinline__ float Silu(float x) { return x * FastRcp(1.0f + FastExp(-x)); }

// GELU, tanh form: 0.5 x (1 + tanh(y)), y = sqrt(2/pi) (x + 0.044715 x^3),
// computed as the identical x / (1 + e^(-2y)) (1 + tanh(y) = 2 / (1 + e^(-2y))):
// five full-rate operations and two transcendentals per element. Saturates
// through the exponential: e^(-2y) -> inf gives -0 for large negative x,
// -> 0 gives x for large positive x.
__device__ __forceinline__ float GeluTanh(float x)
{
    const float c = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
    const float u = 1.0f + 0.044715f * (x * x);
    return x * FastRcp(1.0f + __builtin_amdgcn_exp2f(c * x * u));
}

__device__ __forceinline__ float F16ToF32(uint16_t h)
{
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return float(v);
}

__device__ __forceinline__ uint16_t F32ToF16(float f)
{
    _Float16 v = _Float16(f);  // v_cvt_f16_f32: round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &v, 2);
    return b;
}

template <int DT> struct Elem;
template <> struct Elem<kBF16> {
    __device__ static float Load(uint16_t b) { return BF16ToF32(b); }
    __device__ static uint16_t Store(float f) { return F32ToBF16(f); }
};
template <> struct Elem<kF16> {
    __device__ static float Load(uint16_t b) { return F16ToF32(b); }
    __device__ static uint16_t Store(float f) { return F32ToF16(f); }
};

// Round-trip through the storage type: the value a consumer would read back.
template <int DT>
__device__ __forceinline__ float RoundTo(float f)
{
    return Elem<DT>::Load(Elem<DT>::Store(f));
}

// 16-byte vector of eight 16-bit elements.
struct alignas(16) U16x8 {
    uint16_t v[8];
};

__device__ __forceinline__ U16x8 LoadU16x8(const uint16_t *p)
{
    U16x8 r;
    *reinterpret_cast<uint4 *>(r.v) = *reinterpret_cast<const uint4 *>(p);
    return r;
}

__device__ __forceinline__ void StoreU16x8(uint16_t *p, const U16x8 &r)
{
    *reinterpret_cast<uint4 *>(p) = *reinterpret_cast<const uint4 *>(r.v);
}

// Wavefront-wide reductions (64 lanes) via DPP-backed shuffles.
__device__ __forceinline__ float WaveSum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float WaveMax(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace kr
