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
inline std::vector<uint32_t> ConsumerCuMask(int num_cus, int per_xcd)
{
    std::vector<uint32_t> mask((num_cus + 31) / 32, 0u);
    const int per_xcd_cus = num_cus / 8;
    per_xcd = std::max(1, std::min(per_xcd, per_xcd_cus / 8 > 0 ? 4 : 1));
    for (int x = 0; x < 8; ++x)
        for (int j = 0; j < per_xcd; ++j) {
            const int c = per_xcd_cus * x + ((x + 8 * j) % per_xcd_cus);
            if (c < num_cus) mask[c / 32] |= 1u << (c % 32);
        }
    return mask;
}

// Producer + consumer stream pair, each on its own hardware queue.
//
// The relay waits in both directions on the device (consumer kernels spin on
// producer tiles, the producer's one-workgroup waits spin on consumer
// releases), so the two streams must run concurrently. Ordinary streams are
// multiplexed onto a few hardware queues once a process holds more streams
// than GPU_MAX_HW_QUEUES (a torch stream pool alone creates 32): two streams on
// one queue would run a captured producer graph to completion before the
// consumer graph starts. A CU-masked stream always gets a queue of its own, so
// both streams are created with explicit CU masks: the producer with every
// CU, the consumer with every CU or, with KR_CONSUMER_CUS_PER_XCD = 1..4, a
// few CUs per XCD so spinning consumers can only ever occupy those.
struct StreamPair {
    hipStream_t prod = nullptr;
    hipStream_t cons = nullptr;
    int cons_cus = 0;  // CUs in the consumer mask
    int prod_cus = 0;

    void Create(int device)
    {
        hipDeviceProp_t prop;
        Check(hipGetDeviceProperties(&prop, device), "device props");
        const int ncu = prop.multiProcessorCount;
        std::vector<uint32_t> all((ncu + 31) / 32, 0u);
        for (int c = 0; c < ncu; ++c) all[c / 32] |= 1u << (c % 32);
        Check(hipExtStreamCreateWithCUMask(&prod, uint32_t(all.size()), all.data()), "create producer stream");
        prod_cus = ncu;
        const int per_xcd = EnvInt("KR_CONSUMER_CUS_PER_XCD", 0);
        std::vector<uint32_t> mask = per_xcd > 0 ? ConsumerCuMask(ncu, per_xcd) : all;
        Check(hipExtStreamCreateWithCUMask(&cons, uint32_t(mask.size()), mask.data()), "create consumer stream");
        for (uint32_t w : mask) cons_cus += __builtin_popcount(w);
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
