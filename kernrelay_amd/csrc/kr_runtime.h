// Host-side runtime helpers shared by the schedule executor (kr_plan.cpp)
// and the Qwen prefill runtime (kr_qwen.cpp).
#pragma once

#include <hip/hip_ext.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <string>
#include <vector>

#include "kr_common.h"

namespace kr {

using Clock = std::chrono::steady_clock;

inline double Us(Clock::time_point a, Clock::time_point b)
{
    return std::chrono::duration<double, std::micro>(b - a).count();
}

inline int EnvInt(const char *name, int dflt)
{
    const char *v = std::getenv(name);
    if (v == nullptr || *v == '\0') return dflt;
    return std::atoi(v);
}

inline std::string EnvStr(const char *name, const std::string &dflt)
{
    const char *v = std::getenv(name);
    return (v == nullptr || *v == '\0') ? dflt : std::string(v);
}

// Owning device allocation.
class DevBuf {
public:
    DevBuf() = default;
    explicit DevBuf(size_t bytes) { Alloc(bytes); }
    ~DevBuf() { Free(); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
    DevBuf &operator=(DevBuf &&o) noexcept
    {
        if (this != &o) {
            Free();
            p_ = o.p_;
            n_ = o.n_;
            o.p_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }
    void Alloc(size_t bytes)
    {
        Free();
        if (bytes == 0) return;
        Check(hipMalloc(&p_, bytes), "hipMalloc");
        n_ = bytes;
    }
    void Free()
    {
        if (p_) (void)hipFree(p_);
        p_ = nullptr;
        n_ = 0;
    }
    void *get() const { return p_; }
    template <typename T> T *as() const { return static_cast<T *>(p_); }
    size_t bytes() const { return n_; }

private:
    void *p_ = nullptr;
    size_t n_ = 0;
};

// The reference's deterministic input value (exec/exec_main.cpp:74-79):
// multiples of 1/256 in [-11/256, 11/256], exact in fp16 and bf16.
inline float DetValue(uint32_t seed, size_t index)
{
    const uint32_t h = static_cast<uint32_t>(index) * 2654435761U + seed * 40503U + 7U;
    const int v = static_cast<int>((h >> 8) % 23U) - 11;
    return static_cast<float>(v) * 0.00390625f;
}

// FNV-1a of the node id plus a per-rank offset (exec/exec_main.cpp:491-496).
inline uint32_t NodeSeed(const std::string &id, uint32_t rank)
{
    uint32_t h = 2166136261U;
    for (char c : id) h = (h ^ static_cast<uint8_t>(c)) * 16777619U;
    return h + rank * 7919U;
}

// CU mask that keeps `per_xcd` CUs in each of the 8 XCDs whether the logical
// CU numbering is XCD-major (CU c in XCD c/32) or XCD-interleaved (c % 8):
// c = 32*x + ((x + 8*j) mod 32). Never leaves an XCD without a CU.
// `per_xcd` CUs on every XCD. Workgroups are dealt to the 8 XCDs
// round-robin and each XCD schedules its share on its own CUs, so a CU set
// that missed an XCD would stall that XCD's share of every kernel launched on
// it (the runtime refuses a queue whose mask leaves an XCD empty), and a set
// that took more from one XCD would make it the straggler. On MI355X mask bit
// c addresses XCD c % 8 (then shader engine, then CU within it), so bits
// x + 8j, j < per_xcd, give every XCD per_xcd CUs on different shader
// engines. KR_CU_LAYOUT=blocked assumes bits [x*n/8, (x+1)*n/8) on XCD x.
inline std::vector<uint32_t> ReservedCuMask(int num_cus, int per_xcd)
{
    std::vector<uint32_t> mask((num_cus + 31) / 32, 0u);
    const std::string layout = EnvStr("KR_CU_LAYOUT", "interleaved");
    const int per = num_cus / 8;
    for (int x = 0; x < 8; ++x)
        for (int j = 0; j < per_xcd && j < per; ++j) {
            const int c = layout == "blocked" ? per * x + j : x + 8 * j;
            if (c < num_cus) mask[c / 32] |= 1u << (c % 32);
        }
    return mask;
}

// Producer + consumer stream pair, each on its own hardware queue.
//
// The relay waits in both directions on the device, so the two streams must
// run concurrently. Ordinary streams are multiplexed onto a few hardware
// queues once a process holds more streams than GPU_MAX_HW_QUEUES (a torch
// stream pool alone creates 32): two streams on one queue would run a
// captured producer graph to completion before the consumer graph starts. A
// CU-masked stream always gets a queue of its own, so both streams are
// created with explicit CU masks.
// * partition_per_xcd > 0 (relay split): the consumer owns that many CUs per
//   XCD and the producer the rest, disjoint. A 256x256 GEMM workgroup needs a
//   whole CU; consumer workgroups interleaved onto the producer's CUs keep
//   CUs from draining and starve both kernels, so the two engines get
//   separate CUs as the reference's AIC/AIV cores are separate.
// * Otherwise the producer gets every CU and the consumer every CU or, with
//   KR_CONSUMER_CUS_PER_XCD = 1..4, a few CUs per XCD.
struct StreamPair {
    hipStream_t prod = nullptr;
    hipStream_t cons = nullptr;
    int cons_cus = 0;  // CUs in the consumer mask
    int prod_cus = 0;

    void Create(int device, int partition_per_xcd = 0)
    {
        hipDeviceProp_t prop;
        Check(hipGetDeviceProperties(&prop, device), "device props");
        const int ncu = prop.multiProcessorCount;
        std::vector<uint32_t> all((ncu + 31) / 32, 0u);
        for (int c = 0; c < ncu; ++c) all[c / 32] |= 1u << (c % 32);
        std::vector<uint32_t> pmask = all, cmask = all;
        if (partition_per_xcd > 0) {
            cmask = ReservedCuMask(ncu, partition_per_xcd);
            for (size_t i = 0; i < pmask.size(); ++i) pmask[i] &= ~cmask[i];
        } else if (const int per_xcd = EnvInt("KR_CONSUMER_CUS_PER_XCD", 0); per_xcd > 0) {
            cmask = ReservedCuMask(ncu, std::min(per_xcd, 4));
        }
        Check(hipExtStreamCreateWithCUMask(&prod, uint32_t(pmask.size()), pmask.data()), "create producer stream");
        Check(hipExtStreamCreateWithCUMask(&cons, uint32_t(cmask.size()), cmask.data()), "create consumer stream");
        for (uint32_t w : pmask) prod_cus += __builtin_popcount(w);
        for (uint32_t w : cmask) cons_cus += __builtin_popcount(w);
    }
    void Destroy()
    {
        if (prod) (void)hipStreamDestroy(prod);
        if (cons) (void)hipStreamDestroy(cons);
        prod = cons = nullptr;
    }
};

inline double Median(std::vector<double> v)
{
    if (v.empty()) return 0.0;
    std::sort(v.begin(), v.end());
    const size_t n = v.size();
    return n % 2 ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
}

inline double Min(const std::vector<double> &v) { return v.empty() ? 0.0 : *std::min_element(v.begin(), v.end()); }

}  // namespace kr
