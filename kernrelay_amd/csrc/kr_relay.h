// Device-side relay protocol: monotone counters in HBM.
//
// Control blocks are 32 bytes (8 x int32), laid out as the reference's
// kr::kWords block (kernels/kr_sync_common.h:10-15) with the reference's three
// words first:
//   [0] published  producer: +1 per release of the tile (monotone, never reset)
//   [1] consumed   consumer: advanced by one once it has waited
//   [2] status     consumer: 1 = released in time, 2 = spin bound exceeded
//   [3] arrive     producer workgroup arrival ticket for the pending release
//   [4] done       consumer workgroup completion ticket
//   [5] timed_out  set by any consumer workgroup that exceeded its spin bound
//   [6..7] unused
// A producer tile owns a *flag* block (words 0 and 3). Each consumer of that
// tile owns a *state* block (words 1, 2, 4, 5). For a 1:1 edge both roles use
// the same block, which is exactly the reference's [published, consumed,
// status] edge; a fan-out gives every consumer its own state block while all
// of them spin on the one flag. Because `published` and `consumed` only grow,
// a captured hipGraph replays without the host clearing anything (reference
// kernels/kr_wait_aiv.cpp:19-28 derives target = consumed + 1 the same way).
//
// The reference publishes with a separate kernel after the producer and waits
// with a separate kernel before the consumer (kernels/kr_publish_aiv.cpp:6-23,
// kernels/kr_wait_aiv.cpp:7-36). Here the release is folded into the
// producer's epilogue (every workgroup arrives; the last one releases) and
// the wait into the consumer's prologue (one lane spins on an agent-scope load
// with s_sleep backoff, then a workgroup barrier). Cross-XCD visibility: the
// producer writes released data with device-scope stores and arrives only
// once they are acknowledged (no cache-wide write-back, see RelayArrive); a
// consumer that waits inside its own kernel takes an agent-scope acquire
// (its XCD's caches may hold stale lines of the buffer), and a consumer
// launched behind a wait kernel gets the acquire of its own kernel start.
#pragma once

#include "kr_common.h"

namespace kr {

constexpr int kWords = 8;
constexpr int kOffPublished = 0;
constexpr int kOffConsumed = 1;
constexpr int kOffStatus = 2;
constexpr int kOffArrive = 3;
constexpr int kOffDone = 4;
constexpr int kOffTimedOut = 5;

constexpr uint32_t kDefaultMaxSpins = 1u << 22;

// Consumer side. Row r of this launch is producer row (r + row_off); producer
// tile k covers producer rows [k*prod_rows, (k+1)*prod_rows), its flag is
// block (flag0 + k) and this consumer's state for it is block (state0 + k).
// State blocks adv_lo..adv_hi-1 are consumed (consumed/status advanced) by
// this launch; a launch that waits on a tile a later launch of the same
// consumer also waits on leaves it to that launch (exactly-once consumption
// under m:n row geometry).
struct RelayWait {
    int32_t *ctrl;  // nullptr: no waiting
    int32_t flag0;
    int32_t state0;
    int32_t prod_rows;
    int32_t row_off;
    int32_t adv_lo;
    int32_t adv_hi;
    uint32_t max_spins;
};

// Producer side: tile t = rows [t*rows_per_tile, (t+1)*rows_per_tile) of this
// launch; once `arrivals` workgroups have arrived for it, flag block
// (flag0 + t) is released.
struct RelayPub {
    int32_t *ctrl;  // nullptr: no publishing
    int32_t flag0;
    int32_t rows_per_tile;
    int32_t arrivals;
};

__device__ __forceinline__ int32_t LoadRelaxed(int32_t *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void StoreRelaxed(int32_t *p, int32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One lane: spin until the flag has been published once more than this
// consumer has consumed. On hitting the bound, flag timed_out and go on (the
// reference's wait kernel likewise proceeds and reports status 2).
__device__ __forceinline__ void SpinOnTile(int32_t *flag, int32_t *state, uint32_t max_spins)
{
    const int32_t target = LoadRelaxed(state + kOffConsumed) + 1;
    uint32_t spins = 0;
    while (LoadRelaxed(flag + kOffPublished) < target) {
        if (++spins > max_spins) {
            StoreRelaxed(state + kOffTimedOut, 1);
            return;
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

// Every thread of the workgroup calls this before reading rows [lo, hi) of
// its input (local numbering). Lane 0 spins; the barrier hands the acquire
// to the rest of the workgroup.
__device__ __forceinline__ void RelayWaitRows(const RelayWait &w, int lo, int hi)
{
    if (w.ctrl == nullptr || hi <= lo) return;
    if (threadIdx.x == 0) {
        const int k0 = (lo + w.row_off) / w.prod_rows;
        const int k1 = (hi - 1 + w.row_off) / w.prod_rows;
        for (int k = k0; k <= k1; ++k) {
            SpinOnTile(w.ctrl + size_t(w.flag0 + k) * kWords, w.ctrl + size_t(w.state0 + k) * kWords,
                       w.max_spins);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
}

// Every thread calls this at the very end of a consumer kernel. The last
// workgroup to finish advances `consumed` and writes `status` for the state
// blocks this launch consumes.
__device__ __forceinline__ void RelayFinish(const RelayWait &w)
{
    if (w.ctrl == nullptr || w.adv_hi <= w.adv_lo) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        // relaxed is enough: this workgroup's waits (the loads of `consumed`
        // it spun on) have completed before its ticket, and the counters are
        // next read by waiters of a later launch or by the host.
        int32_t *ticket = w.ctrl + size_t(w.state0 + w.adv_lo) * kWords + kOffDone;
        const int32_t t = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == int32_t(gridDim.x * gridDim.y * gridDim.z) - 1) {
            StoreRelaxed(ticket, 0);
            for (int k = w.adv_lo; k < w.adv_hi; ++k) {
                int32_t *st = w.ctrl + size_t(w.state0 + k) * kWords;
                const int32_t c = LoadRelaxed(st + kOffConsumed);
                const int32_t to =
                    __hip_atomic_exchange(st + kOffTimedOut, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                StoreRelaxed(st + kOffConsumed, c + 1);
                StoreRelaxed(st + kOffStatus, to ? 2 : 1);
            }
        }
    }
}

// RelayFinish for a launch that stands in for several consumers of the same
// producer tiles (sibling consumers fused into one kernel): the state blocks
// of every consumer (bases states[0..n)) advance together over adv_lo..adv_hi.
// w.state0 must equal states[0] (its `done` word is the completion ticket).
__device__ __forceinline__ void RelayFinishMulti(const RelayWait &w, const int32_t *states, int n)
{
    if (w.ctrl == nullptr || w.adv_hi <= w.adv_lo) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t *ticket = w.ctrl + size_t(w.state0 + w.adv_lo) * kWords + kOffDone;
        const int32_t t = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == int32_t(gridDim.x * gridDim.y * gridDim.z) - 1) {
            StoreRelaxed(ticket, 0);
            // a timeout seen by any workgroup is recorded on the first
            // consumer's state (the one the spins read); every fused consumer
            // reports it
            for (int k = w.adv_lo; k < w.adv_hi; ++k) {
                const int32_t to = __hip_atomic_exchange(w.ctrl + size_t(w.state0 + k) * kWords + kOffTimedOut, 0,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int i = 0; i < n; ++i) {
                    int32_t *st = w.ctrl + size_t(states[i] + k) * kWords;
                    StoreRelaxed(st + kOffConsumed, LoadRelaxed(st + kOffConsumed) + 1);
                    StoreRelaxed(st + kOffStatus, to ? 2 : 1);
                }
            }
        }
    }
}

// Stores of data a relay releases. A producer that publishes writes its
// outputs with device-scope stores (sc1: written through this XCD's L2 to
// memory, where every XCD reads it), so a release needs no cache-wide
// operation: an agent-scope release fence would write back the whole L2 of
// the XCD (buffer_wbl2) once per workgroup, and the consumer's matching
// acquire would invalidate the L2 that a concurrently running GEMM relies on
// for operand reuse. Ordinary stores when `coherent` is false (no release).
typedef uint32_t RelayU32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void PutU128(void *p, uint4 v, bool coherent)
{
    if (coherent) {
        const RelayU32x4 w = {v.x, v.y, v.z, v.w};
        // a store of more than 8 bytes reads its data VGPRs after issue: two
        // wait states before anything may overwrite them (the compiler cannot
        // see into the asm to insert them itself)
        asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(w) : "memory");
    } else {
        *reinterpret_cast<uint4 *>(p) = v;
    }
}

__device__ __forceinline__ void PutU32(void *p, uint32_t v, bool coherent)
{
    if (coherent) {
        asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
    } else {
        *reinterpret_cast<uint32_t *>(p) = v;
    }
}

__device__ __forceinline__ void PutU16(void *p, uint16_t v, bool coherent)
{
    if (coherent) {
        asm volatile("global_store_short %0, %1, off sc1" ::"v"(p), "v"(uint32_t(v)) : "memory");
    } else {
        *reinterpret_cast<uint16_t *>(p) = v;
    }
}

// Every thread calls this after issuing its stores for tile `tile` with the
// Put* helpers (coherent = true). Each thread waits until its stores are
// acknowledged at device scope, the barrier makes that true for the whole
// workgroup, then one device-scope atomic arrives; the last arriving
// workgroup releases the tile by bumping `published`.
__device__ __forceinline__ void RelayArrive(const RelayPub &p, int tile)
{
    if (p.ctrl == nullptr) return;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this lane's stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t *flag = p.ctrl + size_t(p.flag0 + tile) * kWords;
        const int32_t t = __hip_atomic_fetch_add(flag + kOffArrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == p.arrivals - 1) {
            StoreRelaxed(flag + kOffArrive, 0);
            __hip_atomic_fetch_add(flag + kOffPublished, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// RelayArrive that also returns to every thread this workgroup's place in
// the tile's arrival order (0 .. arrivals - 1): a consumer run by the
// producer's own workgroups splits its work by it. `slot` is an LDS int of
// the calling kernel.
__device__ __forceinline__ int RelayArriveIndexed(const RelayPub &p, int tile, int *slot)
{
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this lane's stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t *flag = p.ctrl + size_t(p.flag0 + tile) * kWords;
        const int32_t t = __hip_atomic_fetch_add(flag + kOffArrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == p.arrivals - 1) {
            StoreRelaxed(flag + kOffArrive, 0);
            __hip_atomic_fetch_add(flag + kOffPublished, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *slot = t;
    }
    __syncthreads();
    return *slot;
}

}  // namespace kr
