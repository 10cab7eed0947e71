// gfx950 direct-to-LDS loads and the hand-counted waits that go with them
// (shared by the pipelined GEMM and attention).
//
// global_load_lds_dwordx4: the 64 lanes of a wave each fetch 16 bytes from
// their own global address, and the 1 KB lands contiguously in LDS at the
// wave-uniform byte address in M0 (lane i at M0 + 16 i), with no VGPR
// staging. The loads are issued from inline asm, so the compiler does not
// count them: the code that issues them waits with an explicit s_waitcnt
// vmcnt before anything reads the LDS they fill. Nothing else in the kernels
// that use them touches M0.
#pragma once

#include "kr_common.h"

namespace kr {

typedef __attribute__((address_space(3))) void *LdsPtr;

// gfx9 s_waitcnt immediates: vmcnt <= n only; vmcnt <= n and lgkmcnt == 0.
#define KR_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (0x7 << 4) | (0xF << 8) | ((((n) >> 4) & 3) << 14))
#define KR_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (0x7 << 4) | ((((n) >> 4) & 3) << 14))

// LDS byte address of a __shared__ object (what M0 takes)
__device__ __forceinline__ uint32_t LdsAddr(const void *p)
{
    return uint32_t(reinterpret_cast<uintptr_t>((LdsPtr)(const_cast<void *>(p))));
}

__device__ __forceinline__ void DmaLoad16(const void *gptr, uint32_t lds_addr)
{
    // one wait state between the M0 write and the LDS DMA that reads it
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_addr) : "memory");
}

__device__ __forceinline__ void DmaTouch4(const void *gptr, uint32_t lds_addr)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(gptr), "s"(lds_addr) : "memory");
}

}  // namespace kr
