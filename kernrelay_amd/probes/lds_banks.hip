// LDS bank conflicts of ds_read_b128 lane patterns: each dispatch has one
// wave read a 64-lane pattern of 16-byte units 4096 times (one read in
// flight). With
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS --kernel-trace
// SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS per Probe dispatch is the conflict
// cycles per read. Patterns: the GEMM's 32-row and 16-row fragment reads
// (lane l: row l % 32 or l % 16 of 128-byte rows, 16-byte chunk l / 32 or
// l / 16 plus the k step's first chunk, slot chunk ^ swizzle(row)) under
// several row swizzles, and contiguous 1 KB.
//   hipcc -O2 --offload-arch=gfx950 lds_banks.hip -o lds_banks
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

constexpr int kUnits = 2048;  // 32 KB of 16-byte units

__global__ void __launch_bounds__(64) Probe(const int *pat, int *out)
{
    __shared__ uint4 buf[kUnits];
    const int l = threadIdx.x;
    for (int i = l; i < kUnits; i += 64) buf[i] = make_uint4(i, i + 1, i + 2, i + 3);
    __syncthreads();
    const int u = pat[l] & (kUnits - 1);
    const uint32_t addr = uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)(&buf[u])));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    uint32_t x = 0;
    for (int it = 0; it < 4096; ++it) {
        u32x4 v;
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
        x ^= v.x + v.w;
    }
    out[l] = int(x);
}

static int Swizzle(int kind, int r)
{
    switch (kind) {
        case 0: return (r & 7) ^ ((r >> 3) & 1);
        case 1: return r & 7;
        case 2: return (r >> 1) & 7;
        default: return 0;
    }
}

int main()
{
    std::vector<std::vector<int>> pats;
    std::vector<std::string> names;
    std::vector<int> p(64);
    for (int l = 0; l < 64; ++l) p[l] = l;
    names.push_back("contiguous");
    pats.push_back(p);
    const char *sw[] = {"(r&7)^((r>>3)&1)", "r&7", "(r>>1)&7"};
    for (int rows : {32, 16})
        for (int kind = 0; kind < 3; ++kind)
            for (int c0 : {0, 4}) {
                for (int l = 0; l < 64; ++l) {
                    const int r = l % rows, c = c0 + l / rows;
                    p[l] = r * 8 + ((c & 7) ^ Swizzle(kind, r));
                }
                names.push_back(std::to_string(rows) + "-row fragment, chunk " + std::to_string(c0) + ", swizzle " +
                                sw[kind]);
                pats.push_back(p);
            }
    int *dp = nullptr, *dout = nullptr;
    if (hipMalloc(&dp, 64 * 4) != hipSuccess || hipMalloc(&dout, 64 * 4) != hipSuccess) return 1;
    for (size_t i = 0; i < pats.size(); ++i) {
        (void)hipMemcpy(dp, pats[i].data(), 64 * 4, hipMemcpyHostToDevice);
        hipLaunchKernelGGL(Probe, dim3(1), dim3(64), 0, 0, dp, dout);
        (void)hipDeviceSynchronize();
        std::printf("Probe dispatch %zu: %s\n", i + 1, names[i].c_str());
    }
    return 0;
}
