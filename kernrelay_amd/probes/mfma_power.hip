// MFMA-only throughput under the card's power limit: v_mfma_f32_32x32x16_bf16
// against v_mfma_f32_16x16x32_bf16 with the same flops per loop iteration, the
// same accumulator registers (128 per lane) and the same operand toggling
// (4 XORs per iteration, as a refill would change them), on every CU at two
// waves per SIMD. Prints TFLOP/s per run; with
//   rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES
// the clock (GRBM_GUI_ACTIVE / 8 XCDs / duration) and the MFMA busy
// fraction of each shape.
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops mfma_power.hip -o mfma_power
//   ./mfma_power 40000
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWgs = 256;   // one 8-wave workgroup per CU
constexpr int kThr = 512;
constexpr int kIn = 65536;  // 16-byte operand values in the input table

template <int V>
__global__ void __launch_bounds__(kThr) MfmaLoop(const u32x4 *in, float *out, int iters)
{
    const int t = blockIdx.x * kThr + threadIdx.x;
    u32x4 a[4], b[4];
    for (int i = 0; i < 4; ++i) {
        a[i] = in[(t * 8 + i) & (kIn - 1)];
        b[i] = in[(t * 8 + 4 + i) & (kIn - 1)];
    }
    float s = 0.f;
    if constexpr (V == 0) {
        f32x16 acc[8];
        for (int i = 0; i < 8; ++i)
            for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, a[(i + h) & 3]),
                        __builtin_bit_cast(bf16x8, b[(i >> 2) + 2 * ((it + h) & 1)]), acc[i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = a[i] ^ b[(i + it) & 3];
        }
        for (int i = 0; i < 8; ++i)
            for (int e = 0; e < 16; ++e) s += acc[i][e];
    } else {
        f32x4 acc[32];
        for (int i = 0; i < 32; ++i)
            for (int e = 0; e < 4; ++e) acc[i][e] = 0.f;
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, a[i & 3]),
                    __builtin_bit_cast(bf16x8, b[((i >> 3) & 1) + 2 * (it & 1)]), acc[i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = a[i] ^ b[(i + it) & 3];
        }
        for (int i = 0; i < 32; ++i)
            for (int e = 0; e < 4; ++e) s += acc[i][e];
    }
    out[t] = s;
}

int main(int argc, char **argv)
{
    const int iters = argc > 1 ? std::atoi(argv[1]) : 40000;
    // operands: random bf16 values in [1, 2) with random signs
    std::vector<uint32_t> h(kIn * 4);
    uint32_t x = 12345;
    for (auto &v : h) {
        x = x * 1664525u + 1013904223u;
        const uint32_t lo = 0x3f80 | ((x >> 9) & 0x7f) | ((x >> 2) & 0x8000);
        x = x * 1664525u + 1013904223u;
        const uint32_t hi = 0x3f80 | ((x >> 9) & 0x7f) | ((x >> 2) & 0x8000);
        v = lo | (hi << 16);
    }
    u32x4 *din = nullptr;
    float *dout = nullptr;
    if (hipMalloc(&din, size_t(kIn) * 16) != hipSuccess || hipMalloc(&dout, size_t(kWgs) * kThr * 4) != hipSuccess)
        return 1;
    (void)hipMemcpy(din, h.data(), size_t(kIn) * 16, hipMemcpyHostToDevice);
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    for (int rep = 0; rep < 3; ++rep)
        for (int v = 0; v < 2; ++v) {
            auto k = v == 0 ? MfmaLoop<0> : MfmaLoop<1>;
            hipLaunchKernelGGL(k, dim3(kWgs), dim3(kThr), 0, 0, din, dout, iters / 10);
            (void)hipDeviceSynchronize();
            (void)hipEventRecord(e0);
            hipLaunchKernelGGL(k, dim3(kWgs), dim3(kThr), 0, 0, din, dout, iters);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            float ms = 0.f;
            (void)hipEventElapsedTime(&ms, e0, e1);
            const double flops = double(kWgs) * (kThr / 64) * iters * 16 * 32768.0;  // same for both shapes
            std::printf("%s: %.3f ms, %.1f TFLOP/s\n", v == 0 ? "32x32x16" : "16x16x32", ms, flops / ms / 1e9);
        }
    return 0;
}
