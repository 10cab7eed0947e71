// Producer GEMM: C[M,N] = A[M,K] . Bt[N,K]^T (+ bias[N]) on CDNA4 MFMA.
//
// Replaces the reference's aclnnMatmul producer (exec/qwen_main.cpp:499-512,
// exec/runtime/op_impl.cpp:175-201). Weights are re-laid out once at load as
// Bt = weight_t^T ([N,K], K contiguous) so that both operands feed the MFMA
// with one 16-byte load per lane.
//
// * 4 waves in a 2x2 grid (each wave owns (BM/2)x(BN/2) of C), or for
//   256x256 tiles 8 waves in a 2x4 grid (128x64 each, two waves per SIMD), as
//   32x32 accumulator blocks (fp32). The 8-wave register-staged kernels and
//   the simple kernel compute a block as four 16x16 sub-blocks with
//   v_mfma_f32_16x16x32 (4 values per lane each); the 4-wave direct-to-LDS
//   kernels as one block with v_mfma_f32_32x32x16 (16 values per lane). The
//   16x16x32 instruction reads and writes a quarter of the accumulator
//   registers of 32x32x16 per flop; under the card's power limit an
//   MFMA-only loop of it held 2.31 GHz against 1.95-2.10 GHz at the same
//   busy fraction (kernrelay_amd/probes/mfma_power.hip).
// * K is walked in 64-wide steps through a double-buffered LDS stage; global
//   loads of step k+1 are in flight while step k runs on the matrix cores.
// * LDS rows are 128 B (64 elements); the 16-byte chunk index is XOR-swizzled
//   with (row>>1)&7, under which the 16 lanes of a fragment read (16
//   consecutive rows, one chunk) hit distinct banks (0 conflict cycles
//   measured by kernrelay_amd/probes/lds_banks.hip).
// * Every variant walks K in the same order, and the two MFMA shapes give
//   the same bits for the same K order, so a row of C is bit-identical
//   whatever BM/BN or row range a launch covers: the split schedule is
//   bit-exact against the unsplit one.
// * The MFMA is fed (B fragment, A fragment), so each block holds C^T: in a
//   16x16 sub-block lane l owns row l % 16 and columns 4 (l / 16) .. + 3, in
//   a 32x32 block row l % 32 and four runs of 4 columns.
// * Epilogue: acc -> 16-bit (RNE); with bias, bf16(bf16(acc)+bias) — the
//   rounding of the reference's separate Matmul then Add (EmitQkv,
//   exec/qwen_main.cpp:1336-1344). The tile is staged row-major in LDS
//   (8-byte writes, XOR-swizzled) and leaves as full-line 16-byte stores. Then
//   the workgroup arrives on its row tile's relay counter; the last arrival
//   releases the tile.
#include "kr_dma.h"
#include "kr_gemm.h"
#include "kr_relay.h"
#include "kr_rowcore.h"
#include "kr_rowops.h"

namespace kr {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;          // K elements per LDS stage
constexpr int kRowChunks = 8;    // 16-byte chunks per LDS row
constexpr int kThreads = 256;

struct GemmParams {
    const uint16_t *A;
    const uint16_t *Bt;
    uint16_t *C;
    const uint16_t *bias;
    int64_t lda, ldb, ldc;
    int M, N, K;
    int tiles_m, tiles_n;
    int order_rows;  // > 0: dispatch tiles in relay-tile order, this many rows each
    int group_m;     // raster: row blocks per group (0 = all)
    int store_kind;  // 0 device-scope (default), 1 plain, 2 nontemporal
    RelayPub pub;
    RelayWait wait;
    uint16_t *tail_act;  // SwiGLU tail consumer output (nullptr: none)
    int tail_cols;
    uint16_t *epi_act;   // SwiGLU epilogue output [M, N/2] (nullptr: store C)
    int64_t ld_act;
    void *uy;        // unary consumer output (nullptr: none)
    int uop, udt;
    int64_t ldy;
    int sk_wgs;          // stream-K workgroups (0: one tile per workgroup)
    int sk_pmax;         // partial-sum slots per tile in sk_ws
    float *sk_ws;        // [tiles][sk_pmax][BM*BN] fp32 partials
    int32_t *sk_cnt;     // [tiles] arrival counters, zero between launches
    int gemm_wgs;        // workgroups of the GEMM proper; the rest are tail
    int tail_wpt;        // tail workgroups per relay tile
    const uint16_t *rope_cos;  // RoPE epilogue (nullptr: none)
    const uint16_t *rope_sin;
    int rope_cols, rope_d, rope_pos0;
    // Add+RMSNorm relay consumer run by the producer's workgroups (rn_y ==
    // nullptr: none): y = rmsnorm(res + C) * gamma, sum = res + C, per row of
    // every released relay tile; all [M, N] packed
    const uint16_t *rn_res;
    const uint16_t *rn_gamma;
    uint16_t *rn_y;
    uint16_t *rn_sum;
    float *rn_rstd;
    float rn_eps;
    int rn_cpl;          // chunks per lane of a one-wave row (1, 2, 4, 8)
    uint32_t rn_spins;   // spin bound of the wait on a relay tile
};

__device__ __forceinline__ int Swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Workgroup -> output tile. The dispatcher deals workgroups to the 8 XCDs
// round-robin (XCD = blockIdx % 8) and each XCD has its own L2. Within a run
// of `per` consecutive workgroup ids starting at `first`, XCD x takes a
// contiguous chunk of the run's tiles, so a weight column block is read by
// workgroups of one XCD while it sits in that XCD's L2.
// * No relay: one run over all tiles, rastered in groups of group_m row
//   blocks (row blocks fastest within a group), so the tiles an XCD runs at
//   once form a near-square patch of C.
// * Relay (order_rows > 0): one run per relay tile, front to back, so tile 0
//   of the rows is complete first; each run covers order_rows/bm row blocks,
//   odd runs with the weight columns in reverse (each run reads all of the
//   weight, and the blocks the last run read are the ones still cached).

__device__ __forceinline__ void TileOf(int bid, int tiles_m, int tiles_n, int bm, int order_rows, int group_m, int &tm,
                                       int &tn, bool xcd = true)
{
    if (order_rows > 0) {
        const int mt = order_rows / bm;  // row blocks per relay tile
        const int per = mt * tiles_n;
        const int r = bid / per;
        const int t = XcdChunk(bid, r * per, per);
        tm = r * mt + t % mt;
        tn = t / mt;
        // serpentine: odd relay tiles walk the weight columns backwards, so
        // they start on the blocks the previous tile read last (still in MALL)
        if (r & 1) tn = tiles_n - 1 - tn;
        return;
    }
    // grouped raster: runs of `group_m` row blocks fastest, so an XCD's
    // concurrent tiles form a near-square patch (fewer distinct operand
    // slices per K stage in its L2) rather than a tall column
    const int t = xcd ? XcdChunk(bid, 0, tiles_m * tiles_n) : bid;
    const int gm_all = group_m > 0 ? min(group_m, tiles_m) : tiles_m;
    const int per_group = gm_all * tiles_n;
    const int g = t / per_group;
    const int first_m = g * gm_all;
    const int gm = min(tiles_m - first_m, gm_all);
    const int r = t - g * per_group;
    tm = first_m + r % gm;
    tn = r / gm;
}

// One 16x16x32 MFMA on a 16x16 sub-block: a holds 16 rows of the A operand
// (lane l: row l % 16, k 8 (l / 16) .. + 7), b 16 columns of the B operand
// likewise; c: lane l holds column l % 16, rows 4 (l / 16) .. + 3.
template <int DT>
__device__ __forceinline__ f32x4 Mfma(const uint4 &a, const uint4 &b, const f32x4 &c)
{
    if constexpr (DT == kBF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

// One 32x32x16 MFMA on a whole 32x32 block (the direct-to-LDS loop of the
// 4-wave kernels, which measured faster with it): a and b hold 32 rows of
// their operand (lane l: row l % 32, k 8 (l / 32) .. + 7); c: lane l holds
// column l % 32, rows 8 (v / 4) + 4 (l / 32) + v % 4. For the same K order
// it gives the same bits as four 16x16x32 MFMAs over the block's quarters
// (the 7B prefill's logits hash is equal with either).
template <int DT>
__device__ __forceinline__ f32x16 Mfma32(const uint4 &a, const uint4 &b, const f32x16 &c)
{
    if constexpr (DT == kBF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

// Accumulator helpers over both layouts: block (i, j), four-value group c,
// value e (the order stream-K partials are written and read back in).
template <int MI, int NI>
__device__ __forceinline__ void AccZero(f32x4 (&a)[MI][NI][4])
{
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) a[i][j][q][e] = 0.0f;
}
template <int MI, int NI>
__device__ __forceinline__ void AccZero(f32x16 (&a)[MI][NI])
{
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) a[i][j][e] = 0.0f;
}
template <int MI, int NI>
__device__ __forceinline__ float AccAt(const f32x4 (&a)[MI][NI][4], int i, int j, int c, int e)
{
    return a[i][j][c][e];
}
template <int MI, int NI>
__device__ __forceinline__ float AccAt(const f32x16 (&a)[MI][NI], int i, int j, int c, int e)
{
    return a[i][j][4 * c + e];
}
template <int MI, int NI>
__device__ __forceinline__ void AccSet(f32x4 (&a)[MI][NI][4], int i, int j, int c, int e, float v)
{
    a[i][j][c][e] = v;
}
template <int MI, int NI>
__device__ __forceinline__ void AccSet(f32x16 (&a)[MI][NI], int i, int j, int c, int e, float v)
{
    a[i][j][4 * c + e] = v;
}

// ---------------------------------------------------------------- tail
// Gate/up halves of four output chunks of an interleaved gate/up buffer
// (chunk c: 8 gate then 8 up values at c*16), all eight loads device-scope
// (the tile was released by other XCDs' device-scope stores; this XCD's L2
// may hold stale lines of the buffer from an earlier use) and in flight
// together; returns once they have landed.
typedef uint32_t GemmU32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void LoadGateUp4(const uint16_t *p0, const uint16_t *p1, const uint16_t *p2,
                                            const uint16_t *p3, GemmU32x4 (&g)[4], GemmU32x4 (&u)[4])
{
    asm volatile(
        "global_load_dwordx4 %0, %8, off sc1\n\t"
        "global_load_dwordx4 %1, %8, off offset:16 sc1\n\t"
        "global_load_dwordx4 %2, %9, off sc1\n\t"
        "global_load_dwordx4 %3, %9, off offset:16 sc1\n\t"
        "global_load_dwordx4 %4, %10, off sc1\n\t"
        "global_load_dwordx4 %5, %10, off offset:16 sc1\n\t"
        "global_load_dwordx4 %6, %11, off sc1\n\t"
        "global_load_dwordx4 %7, %11, off offset:16 sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(g[0]), "=&v"(u[0]), "=&v"(g[1]), "=&v"(u[1]), "=&v"(g[2]), "=&v"(u[2]), "=&v"(g[3]), "=&v"(u[3])
        : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
        : "memory");
}

// SwiGLU of one chunk, rounded exactly as the standalone kernel rounds it:
// the silu result is stored (16-bit) before the multiply.
template <int DT>
__device__ __forceinline__ uint4 SwigluChunk(const GemmU32x4 &g, const GemmU32x4 &u)
{
    U16x8 a, b, r;
    *reinterpret_cast<GemmU32x4 *>(a.v) = g;
    *reinterpret_cast<GemmU32x4 *>(b.v) = u;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        r.v[e] = Elem<DT>::Store(RoundTo<DT>(Silu(Elem<DT>::Load(a.v[e]))) * Elem<DT>::Load(b.v[e]));
    return *reinterpret_cast<const uint4 *>(r.v);
}

// A tail workgroup: wait for its relay tile, SwiGLU over its share of the
// tile's rows; the last one of the tile consumes the release.
template <int DT>
__device__ void TailSwiglu(const GemmParams &p)
{
    const int j = int(blockIdx.x) - p.gemm_wgs;
    const int t = j / p.tail_wpt;
    const int w = j - t * p.tail_wpt;
    int32_t *flag = p.pub.ctrl + size_t(p.pub.flag0 + t) * kWords;
    if (threadIdx.x == 0) SpinOnTile(flag, flag, kDefaultMaxSpins);
    __syncthreads();
    const int64_t rows = p.pub.rows_per_tile;
    const int64_t chunks = rows * p.tail_cols / 8;
    const uint16_t *src = p.C + int64_t(t) * rows * p.ldc;
    uint16_t *dst = p.tail_act + int64_t(t) * rows * p.tail_cols;
    const int64_t stride = int64_t(p.tail_wpt) * blockDim.x;
    int64_t c = int64_t(w) * blockDim.x + threadIdx.x;
    for (; c + 3 * stride < chunks; c += 4 * stride) {
        GemmU32x4 g[4], u[4];
        LoadGateUp4(src + c * 16, src + (c + stride) * 16, src + (c + 2 * stride) * 16, src + (c + 3 * stride) * 16, g,
                    u);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint4 *>(dst + (c + q * stride) * 8) = SwigluChunk<DT>(g[q], u[q]);
    }
    for (; c < chunks; c += stride) {
        GemmU32x4 g[4], u[4];
        LoadGateUp4(src + c * 16, src + c * 16, src + c * 16, src + c * 16, g, u);
        *reinterpret_cast<uint4 *>(dst + c * 8) = SwigluChunk<DT>(g[0], u[0]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int32_t a = __hip_atomic_fetch_add(flag + kOffDone, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a == p.tail_wpt - 1) {
            StoreRelaxed(flag + kOffDone, 0);
            const int32_t to = __hip_atomic_exchange(flag + kOffTimedOut, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            StoreRelaxed(flag + kOffConsumed, LoadRelaxed(flag + kOffConsumed) + 1);
            StoreRelaxed(flag + kOffStatus, to ? 2 : 1);
        }
    }
}

// ------------------------------------------- Add+RMSNorm relay consumer
// The producer's own workgroups consume its released row tiles (the
// reference's down -> Add+RMSNorm tile loop, exec/qwen_main.cpp:1274-1302,
// without the all-reduce): a workgroup that has stored its C tile and arrived
// on relay tile `tile`'s flag (as the tile's `worker`-th arrival) waits for
// the tile's release (all of its producer workgroups have arrived), then
// computes Add+RMSNorm for rows lo + worker*waves + wave, stepping by
// workers*waves, one row per wave, RB rows' loads in flight at a time, with
// the row code of the standalone row kernel. C is read at device scope
// (written by other XCDs' workgroups of this launch). The last of the tile's
// `workers` consumes the release (consumed + 1, status 1, or 2 when any wait
// ran out of spins). Safe from deadlock because the launcher only asks for
// it when the workgroups a tile waits for are resident together: the whole
// grid, or (dispatched in order, relay tile after relay tile) one relay
// tile's producers.
template <int DT, int CPL, int RB>
__device__ __forceinline__ void NormRows(const GemmParams &p, int lo, int hi, int first, int step)
{
    const int ln = threadIdx.x & 63;
    // a wave's rows are the same for all its lanes: kept in scalar registers,
    // the device-scope loads take their base as a plain buffer resource
    // (a row index the compiler thinks may differ per lane would wrap every
    // load in a loop over the lanes' distinct bases)
    first = __builtin_amdgcn_readfirstlane(first);
    if (lo + first >= hi) return;
    uint4 g[CPL];
    RowGammaLoad<CPL>(p.rn_gamma, p.N, ln, g);
    for (int r0 = lo + first; r0 < hi; r0 += RB * step) {
        RowIn<CPL> in[RB];
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = min(r0 + j * step, hi - 1);  // past the end: re-read, never used
            AddRmsNormLoad<CPL, true>(p.rn_res + int64_t(r) * p.N, p.C + int64_t(r) * p.N, p.N, ln, in[j]);
        }
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = r0 + j * step;
            if (r >= hi) break;
            const int64_t o = int64_t(r) * p.N;
            AddRmsNormFinish<DT, CPL>(in[j], g, p.rn_y + o, p.rn_sum != nullptr ? p.rn_sum + o : nullptr,
                                      p.rn_rstd != nullptr ? p.rn_rstd + r : nullptr, p.N, p.rn_eps, ln, false);
        }
    }
}

template <int DT, int NW, int WPE>
__device__ void NormTail(const GemmParams &p, int tile, int worker, int workers)
{
    int32_t *flag = p.pub.ctrl + size_t(p.pub.flag0 + tile) * kWords;
    if (threadIdx.x == 0) SpinOnTile(flag, flag, p.rn_spins);
    __syncthreads();
    const int R = p.pub.rows_per_tile;
    const int lo = tile * R, hi = min(lo + R, p.M);
    const int first = worker * NW + int(threadIdx.x >> 6);
    const int step = workers * NW;
    // rows in flight per wave: what the registers hold without spilling
    // (WPE waves per SIMD share its 512 registers; loads land in the 256
    // architectural ones)
    constexpr int RB4 = WPE == 2 ? 2 : 4;
    constexpr int RB8 = WPE == 2 ? 1 : 2;
    switch (p.rn_cpl) {
        case 1: NormRows<DT, 1, RB4>(p, lo, hi, first, step); break;
        case 2: NormRows<DT, 2, RB4>(p, lo, hi, first, step); break;
        case 4: NormRows<DT, 4, RB4>(p, lo, hi, first, step); break;
        default: NormRows<DT, 8, RB8>(p, lo, hi, first, step); break;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int32_t a = __hip_atomic_fetch_add(flag + kOffDone, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a == workers - 1) {
            StoreRelaxed(flag + kOffDone, 0);
            const int32_t to = __hip_atomic_exchange(flag + kOffTimedOut, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            StoreRelaxed(flag + kOffConsumed, LoadRelaxed(flag + kOffConsumed) + 1);
            StoreRelaxed(flag + kOffStatus, to ? 2 : 1);
        }
    }
}

// The unary consumer's pass over the staged tile (after C's): y = f(C) with
// the elementwise kernel's arithmetic on C's stored values, so y equals what
// that kernel computes from C bit for bit. Every thread stores 16 bytes of y
// per step -- 8 values of a 16-bit y, 4 of an fp32 y -- so each store
// instruction covers whole 128-byte lines (two 16-byte halves of 32-byte
// runs would leave every line half-written per instruction). Staged chunk c
// of a row sits in slot c ^ ((row & 31) >> 1), its 8-byte halves swapped on
// odd rows. Columns past N are not written.
template <int DT, int BM, int BN, int NT, int OP, int ODT>
__device__ __forceinline__ void UnaryTileOp(const GemmParams &p, const uint16_t *stage, int m0, int n0, bool coh)
{
    auto f = [](uint16_t h) {
        const float x = Elem<DT>::Load(h);
        if constexpr (OP == kEwGelu) {
            return GeluTanh(x);
        } else if constexpr (OP == kEwSilu) {
            return Silu(x);
        } else {
            return x;
        }
    };
    if constexpr (ODT == kF32) {
        constexpr int QPR = BN / 4;  // 4-value quarters per row
#pragma unroll 4
        for (int idx = threadIdx.x; idx < BM * QPR; idx += NT) {
            const int row = idx / QPR;
            const int q = idx % QPR;
            const int gm = m0 + row;
            const int gn = n0 + q * 4;
            if (gm >= p.M || gn >= p.N) continue;
            const int slot = (q >> 1) ^ ((row & 31) >> 1);
            const uint2 u = *reinterpret_cast<const uint2 *>(stage + row * BN + slot * 8 + 4 * ((q ^ row) & 1));
            const float o[4] = {f(uint16_t(u.x)), f(uint16_t(u.x >> 16)), f(uint16_t(u.y)), f(uint16_t(u.y >> 16))};
            float *yp = static_cast<float *>(p.uy) + int64_t(gm) * p.ldy + gn;
            if (gn + 4 <= p.N) {
                PutU128(yp, make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                       __float_as_uint(o[3])), coh);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gn + e < p.N) PutU32(yp + e, __float_as_uint(o[e]), coh);
            }
        }
    } else {
        constexpr int CPR = BN / 8;
#pragma unroll 4
        for (int idx = threadIdx.x; idx < BM * CPR; idx += NT) {
            const int row = idx / CPR;
            const int ch = idx % CPR;
            const int gm = m0 + row;
            const int gn = n0 + ch * 8;
            if (gm >= p.M || gn >= p.N) continue;
            uint4 u = *reinterpret_cast<const uint4 *>(stage + row * BN + (ch ^ ((row & 31) >> 1)) * 8);
            if (row & 1) u = make_uint4(u.z, u.w, u.x, u.y);
            U16x8 a, r;
            *reinterpret_cast<uint4 *>(a.v) = u;
#pragma unroll
            for (int e = 0; e < 8; ++e) r.v[e] = Elem<ODT>::Store(f(a.v[e]));
            uint16_t *yp = static_cast<uint16_t *>(p.uy) + int64_t(gm) * p.ldy + gn;
            if (gn + 8 <= p.N) {
                PutU128(yp, *reinterpret_cast<const uint4 *>(r.v), coh);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (gn + e < p.N) PutU16(yp + e, r.v[e], coh);
            }
        }
    }
}

// The op and output type are the same for the whole launch: one specialised
// loop each, dispatched once per tile. Tested at run time inside the
// element loop, they turned every element into its own small block behind
// uniform branches, its conversion, exponential and reciprocal chain
// overlapping no other element's (the mm -> GELU epilogue took 190 instead
// of 174 us).
template <int DT, int BM, int BN, int NT>
__device__ __forceinline__ void UnaryTile(const GemmParams &p, const uint16_t *stage, int m0, int n0, bool coh)
{
    auto run = [&](auto op) __attribute__((always_inline)) {
        constexpr int OP = decltype(op)::value;
        if (p.udt == kF32) {
            UnaryTileOp<DT, BM, BN, NT, OP, kF32>(p, stage, m0, n0, coh);
        } else if (p.udt == kBF16) {
            UnaryTileOp<DT, BM, BN, NT, OP, kBF16>(p, stage, m0, n0, coh);
        } else {
            UnaryTileOp<DT, BM, BN, NT, OP, kF16>(p, stage, m0, n0, coh);
        }
    };
    if (p.uop == kEwGelu) {
        run(std::integral_constant<int, kEwGelu>{});
    } else if (p.uop == kEwSilu) {
        run(std::integral_constant<int, kEwSilu>{});
    } else {
        run(std::integral_constant<int, kEwCast>{});
    }
}

// Stage the workgroup's BMxBN tile of C in LDS. acc[i][j][2 sn + sm] is the
// C^T 16x16 sub-block of rows wm*BM/2 + 32i + 16sm.., cols wn*BN/2 + 32j +
// 16sn..: value e of lane l sits at row l%16, col 4*(l/16) + e. Each run of
// 4 columns goes to LDS as one 8-byte write into a row-major tile whose
// 8-byte slots are XOR-swizzled with row & 31 (the rows of one column run hit
// distinct bank pairs). `stage` must hold BM*BN 16-bit values and be free
// (all waves past their last LDS read of the main loop).
template <int DT, int BM, int BN, int MI, int NI>
__device__ __forceinline__ void StageTile(const GemmParams &p, f32x4 (&acc)[MI][NI][4], uint16_t *stage, int n0, int wm,
                                          int wn, int lane)
{
    constexpr int WTN = NI * 32;  // columns per wave
    static_assert(BN >= 128, "slot swizzle needs >= 32 slots per row");
    const int lr = lane & 15;         // row in a 16x16 sub-block
    const int lc = 4 * (lane >> 4);   // first of the lane's four columns in it
#pragma unroll
    for (int j = 0; j < NI; ++j) {
#pragma unroll
        for (int sn = 0; sn < 2; ++sn) {
            const int col = wn * WTN + j * 32 + 16 * sn + lc;
            float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (p.bias != nullptr) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n0 + col + e < p.N) b[e] = Elem<DT>::Load(p.bias[n0 + col + e]);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int sm = 0; sm < 2; ++sm) {
                    const int row = wm * (BM / 2) + i * 32 + 16 * sm + lr;
                    uint32_t h[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x = acc[i][j][2 * sn + sm][e];
                        h[e] = p.bias != nullptr ? Elem<DT>::Store(RoundTo<DT>(x) + b[e]) : Elem<DT>::Store(x);
                    }
                    const int slot = (col >> 2) ^ (row & 31);
                    *reinterpret_cast<uint2 *>(stage + row * BN + slot * 4) =
                        make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                }
        }
    }
}

// The same for a 32x32 accumulator block (lane l: row l % 32, four runs of
// 4 consecutive columns 8 g + 4 (l / 32) ..).
template <int DT, int BM, int BN, int MI, int NI>
__device__ __forceinline__ void StageTile(const GemmParams &p, f32x16 (&acc)[MI][NI], uint16_t *stage, int n0, int wm,
                                          int wn, int lane)
{
    constexpr int WTN = NI * 32;  // columns per wave
    static_assert(BN >= 128, "slot swizzle needs >= 32 slots per row");
    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int col = wn * WTN + j * 32 + 8 * g + 4 * lhalf;
            float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (p.bias != nullptr) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n0 + col + e < p.N) b[e] = Elem<DT>::Load(p.bias[n0 + col + e]);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = wm * (BM / 2) + i * 32 + lrow;
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float x = acc[i][j][4 * g + e];
                    h[e] = p.bias != nullptr ? Elem<DT>::Store(RoundTo<DT>(x) + b[e]) : Elem<DT>::Store(x);
                }
                const int slot = (col >> 2) ^ (row & 31);
                *reinterpret_cast<uint2 *>(stage + row * BN + slot * 4) =
                    make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            }
        }
    }
}

// Write the workgroup's BMxBN tile of C: stage it, then every thread copies
// 16-byte row chunks to C (8 lanes cover a 128-byte line), with
// device-scope stores when the launch releases relay tiles.
template <int DT, int BM, int BN, int NT, class ACC>
__device__ __forceinline__ void StoreTile(const GemmParams &p, ACC &acc, uint16_t *stage, int m0, int n0, int wm,
                                          int wn, int lane)
{
    StageTile<DT, BM, BN>(p, acc, stage, n0, wm, wn, lane);
    __syncthreads();
    constexpr int CPR = BN / 8;  // 16-byte chunks per row
    const bool vec = (p.ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0);
    // device-scope stores always: released tiles need them, and written
    // through they also keep the output from evicting the operand tiles the
    // other workgroups of this XCD are still reading from L2
    // (KR_GEMM_STORE=plain|nt for comparison)
    const bool coh = p.store_kind == 0 || p.pub.ctrl != nullptr;
#pragma unroll 4
    for (int idx = threadIdx.x; idx < BM * CPR; idx += NT) {
        const int row = idx / CPR;
        const int ch = idx % CPR;
        const int gm = m0 + row;
        const int gn = n0 + ch * 8;
        if (gm >= p.M || gn >= p.N) continue;
        auto staged = [&](int c) {
            uint4 u = *reinterpret_cast<const uint4 *>(stage + row * BN + (c ^ ((row & 31) >> 1)) * 8);
            return (row & 1) ? make_uint4(u.z, u.w, u.x, u.y) : u;
        };
        uint4 v = staged(ch);
        if (p.rope_cos != nullptr && gn < p.rope_cols) {
            // the partner half of the head is in this tile (tiles start on
            // head boundaries: BN and n0 are multiples of rope_d)
            const int d0 = gn % p.rope_d, half = p.rope_d / 2;
            const uint4 w = staged(d0 < half ? ch + half / 8 : ch - half / 8);
            const int64_t t = int64_t(p.rope_pos0 + gm) * p.rope_d + d0;
            const U16x8 c8 = LoadU16x8(p.rope_cos + t), s8 = LoadU16x8(p.rope_sin + t);
            const uint32_t xv[4] = {v.x, v.y, v.z, v.w}, wv[4] = {w.x, w.y, w.z, w.w};
            uint32_t o[4];
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
                uint32_t pair = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int e = 2 * e2 + h;
                    const float x = Elem<DT>::Load(uint16_t(xv[e2] >> (16 * h)));
                    const float y = Elem<DT>::Load(uint16_t(wv[e2] >> (16 * h)));
                    const float c = Elem<DT>::Load(c8.v[e]), sn = Elem<DT>::Load(s8.v[e]);
                    const float r = d0 < half ? RopeFirst(x, y, c, sn) : RopeSecond(x, y, c, sn);
                    pair |= uint32_t(Elem<DT>::Store(r)) << (16 * h);
                }
                o[e2] = pair;
            }
            v = make_uint4(o[0], o[1], o[2], o[3]);
        }
        uint16_t *dst = p.C + int64_t(gm) * p.ldc + gn;
        if (vec && gn + 8 <= p.N) {
            if (!coh && p.store_kind == 2) {
                __builtin_nontemporal_store(*reinterpret_cast<const RelayU32x4 *>(&v), reinterpret_cast<RelayU32x4 *>(dst));
            } else {
                PutU128(dst, v, coh);
            }
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (gn + e < p.N) PutU16(dst + e, uint16_t(w[e >> 1] >> ((e & 1) * 16)), coh);
        }
    }
    if (p.uy != nullptr) UnaryTile<DT, BM, BN, NT>(p, stage, m0, n0, coh);
}

// SwiGLU epilogue: the in-register relay of the gate/up GEMM to its
// consumer. C's columns hold gate and up interleaved in groups of 8 (cols
// 16q..16q+7 gate, 16q+8..16q+15 up), so a 16x16 C^T sub-block is one group:
// lanes 0-31 hold its gate columns 4 (l / 16) + e, lanes 32-63 the matching
// up columns of the same rows. One v_permlane32_swap per value pairs them
// (lanes 0-31 then hold gate and up of the sub-block's rows 0-15 of sm = 0,
// lanes 32-63 those of sm = 1): act[row, 8q + 4 ((l / 16) & 1) + e] =
// bf16(bf16(silu(bf16(gate))) * bf16(up)), the rounding of the standalone
// SwiGLU kernel reading the stored gate/up tile. C itself is not written.
// The BM x BN/2 act tile is staged in LDS like StoreTile's and leaves as
// full-line 16-byte stores.
template <int DT, int BM, int BN, int MI, int NI>
__device__ __forceinline__ void StageSwiglu(f32x4 (&acc)[MI][NI][4], uint16_t *stage, int wm, int wn, int lane)
{
    constexpr int AW = BN / 2;  // act columns of the tile
    constexpr int WTA = NI * 16;  // act columns per wave
    static_assert(AW >= 128, "slot swizzle needs >= 32 slots per row");
    const int lr = lane & 15;
    const int hi = lane >> 5;                // after the swap: sub-block rows 16 hi ..
    const int lc = 4 * ((lane >> 4) & 1);    // first act column of the lane in its group
#pragma unroll
    for (int j = 0; j < NI; ++j) {
#pragma unroll
        for (int sn = 0; sn < 2; ++sn) {
            const int acol = wn * WTA + j * 16 + 8 * sn + lc;
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = wm * (BM / 2) + i * 32 + 16 * hi + lr;
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[i][j][2 * sn][e]),
                                                                     __float_as_uint(acc[i][j][2 * sn + 1][e]), false,
                                                                     false);
                    const float g = RoundTo<DT>(__uint_as_float(sw[0]));
                    const float u = RoundTo<DT>(__uint_as_float(sw[1]));
                    h[e] = Elem<DT>::Store(RoundTo<DT>(Silu(g)) * u);
                }
                const int slot = (acol >> 2) ^ (row & 31);
                *reinterpret_cast<uint2 *>(stage + row * AW + slot * 4) =
                    make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            }
        }
    }
}

// The same for 32x32 accumulator blocks: a lane's values v = 0..3 are gate
// columns 8g'+4h+e of group q (g' = 2q) and v = 4..7 the matching up
// columns (g' = 2q + 1), so no lane exchange is needed.
template <int DT, int BM, int BN, int MI, int NI>
__device__ __forceinline__ void StageSwiglu(f32x16 (&acc)[MI][NI], uint16_t *stage, int wm, int wn, int lane)
{
    constexpr int AW = BN / 2;  // act columns of the tile
    constexpr int WTA = NI * 16;  // act columns per wave
    static_assert(AW >= 128, "slot swizzle needs >= 32 slots per row");
    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int acol = wn * WTA + j * 16 + q * 8 + 4 * lhalf;
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = wm * (BM / 2) + i * 32 + lrow;
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float g = RoundTo<DT>(acc[i][j][8 * q + e]);
                    const float u = RoundTo<DT>(acc[i][j][8 * q + 4 + e]);
                    h[e] = Elem<DT>::Store(RoundTo<DT>(Silu(g)) * u);
                }
                const int slot = (acol >> 2) ^ (row & 31);
                *reinterpret_cast<uint2 *>(stage + row * AW + slot * 4) =
                    make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            }
        }
    }
}

template <int DT, int BM, int BN, int NT, class ACC>
__device__ __forceinline__ void StoreTileSwiglu(const GemmParams &p, ACC &acc, uint16_t *stage, int m0, int n0, int wm,
                                                int wn, int lane)
{
    constexpr int AW = BN / 2;  // act columns of the tile
    StageSwiglu<DT, BM, BN>(acc, stage, wm, wn, lane);
    __syncthreads();
    constexpr int CPR = AW / 8;
    const int64_t a0 = n0 / 2;
    const int acols = p.N / 2;
#pragma unroll 4
    for (int idx = threadIdx.x; idx < BM * CPR; idx += NT) {
        const int row = idx / CPR;
        const int ch = idx % CPR;
        const int gm = m0 + row;
        const int gn = int(a0) + ch * 8;
        if (gm >= p.M || gn >= acols) continue;
        uint4 v = *reinterpret_cast<const uint4 *>(stage + row * AW + (ch ^ ((row & 31) >> 1)) * 8);
        if (row & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        PutU128(p.epi_act + int64_t(gm) * p.ld_act + gn, v, p.store_kind == 0 || p.pub.ctrl != nullptr);
    }
}

template <int DT, int BM, int BN>
__global__ void __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                               amdgpu_waves_per_eu(BM * BN >= 256 * 128 ? 1 : 2, BM * BN >= 256 * 128 ? 1 : 2)))
GemmKernel(GemmParams p)
{
    constexpr int MI = BM / 64;   // 32-row blocks per wave
    constexpr int NI = BN / 64;   // 32-col blocks per wave
    constexpr int AL = BM * kRowChunks / kThreads;  // A chunks per thread per stage
    constexpr int BL = BN * kRowChunks / kThreads;
    constexpr int STAGE = (BM + BN) * kBK;           // elements per LDS stage

    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];

    if (int(blockIdx.x) >= p.gemm_wgs) {
        TailSwiglu<DT>(p);
        return;
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;

    int tm, tn;
    TileOf(blockIdx.x, p.tiles_m, p.tiles_n, BM, p.order_rows, p.group_m, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    RelayWaitRows(p.wait, m0, min(m0 + BM, p.M));

    const int lrow = tid >> 3;       // 0..31
    const int lchunk = tid & 7;

    uint4 ra[AL], rb[BL];

    auto load_global = [&](int kt) {
        const int kc = kt * kBK + lchunk * 8;
        const bool kin = kc < p.K;
#pragma unroll
        for (int j = 0; j < AL; ++j) {
            const int r = lrow + 32 * j;
            const int gm = m0 + r;
            if (kin && gm < p.M) {
                ra[j] = *reinterpret_cast<const uint4 *>(p.A + int64_t(gm) * p.lda + kc);
            } else {
                ra[j] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < BL; ++j) {
            const int r = lrow + 32 * j;
            const int gn = n0 + r;
            if (kin && gn < p.N) {
                rb[j] = *reinterpret_cast<const uint4 *>(p.Bt + int64_t(gn) * p.ldb + kc);
            } else {
                rb[j] = make_uint4(0, 0, 0, 0);
            }
        }
    };

    auto store_lds = [&](int stage) {
        uint16_t *As = smem + stage * STAGE;
        uint16_t *Bs = As + BM * kBK;
#pragma unroll
        for (int j = 0; j < AL; ++j) {
            const int r = lrow + 32 * j;
            *reinterpret_cast<uint4 *>(As + r * kBK + Swz(r, lchunk) * 8) = ra[j];
        }
#pragma unroll
        for (int j = 0; j < BL; ++j) {
            const int r = lrow + 32 * j;
            *reinterpret_cast<uint4 *>(Bs + r * kBK + Swz(r, lchunk) * 8) = rb[j];
        }
    };

    f32x4 acc[MI][NI][4];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][j][q][v] = 0.0f;

    const int nk = (p.K + kBK - 1) / kBK;
    load_global(0);
    store_lds(0);
    __syncthreads();

    const int frow = lane & 15;
    const int fq = lane >> 4;

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_global(kt + 1);
        const uint16_t *As = smem + cur * STAGE;
        const uint16_t *Bs = As + BM * kBK;
        // two k32 steps: lane l reads row l % 16 of each 16-row fragment,
        // 16-byte chunk 4 ks + l / 16
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ++ks) {
            const int chunk = ks * 4 + fq;
            uint4 fa[MI][2], fb[NI][2];
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int sm = 0; sm < 2; ++sm) {
                    const int r = wm * (BM / 2) + i * 32 + 16 * sm + frow;
                    fa[i][sm] = *reinterpret_cast<const uint4 *>(As + r * kBK + Swz(r, chunk) * 8);
                }
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int sn = 0; sn < 2; ++sn) {
                    const int r = wn * (BN / 2) + j * 32 + 16 * sn + frow;
                    fb[j][sn] = *reinterpret_cast<const uint4 *>(Bs + r * kBK + Swz(r, chunk) * 8);
                }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[i][j][q] = Mfma<DT>(fb[j][q >> 1], fa[i][q & 1], acc[i][j][q]);
        }
        if (kt + 1 < nk) store_lds(cur ^ 1);
        __syncthreads();
    }

    if constexpr (BN >= 256) {
        if (p.epi_act != nullptr) {
            StoreTileSwiglu<DT, BM, BN, kThreads>(p, acc, smem, m0, n0, wm, wn, lane);
        } else {
            StoreTile<DT, BM, BN, kThreads>(p, acc, smem, m0, n0, wm, wn, lane);
        }
    } else {
        StoreTile<DT, BM, BN, kThreads>(p, acc, smem, m0, n0, wm, wn, lane);
    }
    if (p.pub.ctrl != nullptr) {
        const int tile = m0 / p.pub.rows_per_tile;
        const int a = RelayArriveIndexed(p.pub, tile, reinterpret_cast<int *>(smem));  // the tile stage is free
        if (p.rn_y != nullptr) NormTail<DT, kThreads / 64, BM * BN >= 256 * 128 ? 1 : 2>(p, tile, a, p.pub.arrivals);
    }
    RelayFinish(p.wait);
}

// Stream-K partial sums move as 16-byte device-scope accesses (written
// through to memory / read past this XCD's L2, which may hold stale lines of
// the workspace from an earlier launch).
__device__ __forceinline__ void PutF32x4Dev(float *p, float a, float b, float c, float d)
{
    const RelayU32x4 w = {__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)};
    // two wait states before the data VGPRs may be rewritten (as PutU128)
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(w) : "memory");
}

// Eight 16-byte device-scope loads p + u * stride (floats), in flight
// together; returns once all have landed.
__device__ __forceinline__ void GetF32x4x8Dev(const float *p, int64_t stride, RelayU32x4 (&r)[8])
{
    asm volatile(
        "global_load_dwordx4 %0, %8, off sc1\n\t"
        "global_load_dwordx4 %1, %9, off sc1\n\t"
        "global_load_dwordx4 %2, %10, off sc1\n\t"
        "global_load_dwordx4 %3, %11, off sc1\n\t"
        "global_load_dwordx4 %4, %12, off sc1\n\t"
        "global_load_dwordx4 %5, %13, off sc1\n\t"
        "global_load_dwordx4 %6, %14, off sc1\n\t"
        "global_load_dwordx4 %7, %15, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
        : "v"(p), "v"(p + stride), "v"(p + 2 * stride), "v"(p + 3 * stride), "v"(p + 4 * stride),
          "v"(p + 5 * stride), "v"(p + 6 * stride), "v"(p + 7 * stride)
        : "memory");
}

// ---------------------------------------------------------------------------
#include "kr_gemm_pipe.inc"

// KR_GEMM_SIMPLE=1 routes every shape through GemmKernel (A/B comparison of
// the two main loops; both give identical bits).
bool ForceSimple()
{
    static const bool v = [] {
        const char *e = std::getenv("KR_GEMM_SIMPLE");
        return e != nullptr && *e == '1';
    }();
    return v;
}

int StoreKind()
{
    static const int v = [] {
        const char *e = std::getenv("KR_GEMM_STORE");
        if (e == nullptr) return 0;
        return std::string(e) == "plain" ? 1 : std::string(e) == "nt" ? 2 : 0;
    }();
    return v;
}

// Row blocks per raster group of a launch without relay order
// (KR_GEMM_GROUP_M, default 4; 0 = all rows, a column at a time); it changes
// timing only, never the bits.
int RasterGroupM()
{
    static const int v = [] {
        const char *e = std::getenv("KR_GEMM_GROUP_M");
        return e != nullptr ? std::max(0, std::atoi(e)) : 4;
    }();
    return v;
}

// Waves per workgroup of the 256x256 pipelined kernel (KR_GEMM_WAVES: 8
// default, two per SIMD; 4 = one per SIMD); it changes timing only, never
// the bits. Measured on MI355X (cold operands): 4096^3 138 -> 130 us, the
// 2048x4608x3584 QKV 112 -> 104 us, lm_head 2068 -> 2036 us.
int PipeWaves()
{
    static const int v = [] {
        const char *e = std::getenv("KR_GEMM_WAVES");
        return e != nullptr && std::atoi(e) == 4 ? 4 : 8;
    }();
    return v;
}

// Main loop of the 8-wave 256x256 kernel (KR_GEMM_LOOP): 2 (default) =
// register-staged refills spread evenly over each stage, 0 = two 64-deep
// direct-to-LDS stages refilled in a burst after each stage's barrier.
// Timing only, never the bits. Measured on MI355X (us, 0 / 2): 4096^3
// 126.7 / 118.5, gate/up 2048x37888x3584 561 / 529, QKV 2048x4608x3584
// 103 / 85, lm_head 2048x152064x3584 1967 / 1871. Two other schedules
// measured slower than both: the two waves of a SIMD alternating memory and
// MFMA phases on a direct-to-LDS ring (4096^3 140 us), and a ring of four or
// five 32-deep direct-to-LDS stages (142 us: half-line requests). The same
// alternation on the staged refill (per k32 step: fragment reads and half a
// stage of refill, then 32 MFMAs, a barrier after each phase) gave the same
// bits in the same time (4096^3 111.0 against 110.1 us). The 4-wave 256x128 and
// 128x256 kernels keep their three-stage direct-to-LDS ring, which already
// spreads its refills: staged, they measured 4-8% slower.
int MainLoopMode()
{
    static const int v = [] {
        const char *e = std::getenv("KR_GEMM_LOOP");
        return e != nullptr && std::atoi(e) == 0 ? 0 : 2;
    }();
    return v;
}

// L2 prefetch distance of the pipelined kernel in K stages (KR_GEMM_PF: 0
// default = off, 2, 4); it changes timing only, never the bits.
int PrefetchStages()
{
    static const int v = [] {
        const char *e = std::getenv("KR_GEMM_PF");
        return e != nullptr ? std::atoi(e) : 0;
    }();
    return v;
}

// Stream-K plan of a launch: G resident workgroups over tiles x nk
// iterations, at most pmax pieces per tile.
struct StreamKPlan {
    int G = 0, tiles = 0, nk = 0, pmax = 0;
};

int CuCount()
{
    static const int v = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 256;
        return n > 0 ? n : 256;
    }();
    return v;
}

using GemmFn = void (*)(GemmParams);

// The kernel a launch of BM x BN tiles runs over K, and its block size: the
// 8-wave staged kernel for 192x256; for 256x256 the 8-wave kernel (stream-K
// or data-parallel) unless KR_GEMM_WAVES=4; the 4-wave pipelined kernel for
// the other tiles; the simple kernel where K % 64 != 0 or KR_GEMM_SIMPLE=1.
template <int DT, int BM, int BN>
GemmFn PickGemmKernel(int K, bool sk, int &threads)
{
    if constexpr (BM == 192) {
        // 192x256: the 8-wave staged kernel only (GemmLaunch picks this tile
        // only where that kernel runs)
        static_assert(BN == 256, "192-row tiles pair with 256 columns");
        if (sk || K % kPipeK != 0 || ForceSimple() || MainLoopMode() != 2)
            throw std::logic_error("gemm: 192x256 tiles run the staged kernel only");
        threads = 512;
        return GemmPipeKernel<DT, BM, BN, 0, 8, false, 2>;
    } else {
        if (K % kPipeK == 0 && !ForceSimple()) {
            if constexpr (BM == 256 && BN == 256) {
                if (sk) {
                    threads = 512;
                    return MainLoopMode() == 2 ? GemmPipeKernel<DT, BM, BN, 0, 8, true, 2>
                                               : GemmPipeKernel<DT, BM, BN, 0, 8, true>;
                }
                if (PipeWaves() == 8) {
                    threads = 512;
                    return MainLoopMode() == 2 ? GemmPipeKernel<DT, BM, BN, 0, 8, false, 2>
                                               : GemmPipeKernel<DT, BM, BN, 0, 8>;
                }
            }
            threads = kThreads;
            switch (PrefetchStages()) {
            case 2: return GemmPipeKernel<DT, BM, BN, 2, 4>;
            case 4: return GemmPipeKernel<DT, BM, BN, 4, 4>;
            default: return GemmPipeKernel<DT, BM, BN, 0, 4>;
            }
        }
        threads = kThreads;
        return GemmKernel<DT, BM, BN>;
    }
}

// Workgroups of that kernel one CU holds at once, from the runtime's
// occupancy query on the exact instantiation (registers, LDS, waves);
// cached per (dtype, tile, K-path, stream-K).
template <int DT, int BM, int BN>
int GemmWgsPerCu(int K, bool sk)
{
    static int cache[2][2] = {{-1, -1}, {-1, -1}};
    int &c = cache[K % kPipeK == 0 ? 1 : 0][sk ? 1 : 0];
    if (c < 0) {
        int threads = 0;
        const GemmFn fn = PickGemmKernel<DT, BM, BN>(K, sk, threads);
        int n = 0;
        Check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(fn), threads, 0),
              "gemm occupancy");
        if (n < 1) throw std::runtime_error("gemm: kernel does not fit a CU");
        c = n;
    }
    return c;
}

int GemmWgsPerCu(int dt, int bm, int bn, int K, bool sk)
{
    const bool bf = dt == kBF16;
#define KR_OCC_CASE(BM_, BN_) \
    if (bm == BM_ && bn == BN_) return bf ? GemmWgsPerCu<kBF16, BM_, BN_>(K, sk) : GemmWgsPerCu<kF16, BM_, BN_>(K, sk);
    KR_OCC_CASE(256, 256)
    KR_OCC_CASE(192, 256)
    KR_OCC_CASE(256, 128)
    KR_OCC_CASE(128, 256)
    KR_OCC_CASE(128, 128)
    KR_OCC_CASE(64, 256)
#undef KR_OCC_CASE
    throw std::runtime_error("gemm: unsupported tile " + std::to_string(bm) + "x" + std::to_string(bn));
}

// The Add+RMSNorm relay consumer waits inside the producer's workgroups for
// the other producer workgroups of its relay tile. Workgroups are dispatched
// in id order (per XCD) and a relay tile's are consecutive ids, so the waits
// always end when a relay tile's workgroups fit the device at once: then
// every earlier tile's workgroups are resident or finished. A stream-K grid
// must be resident as a whole. The device's slots come from the occupancy of
// the kernel the launch runs.
bool NormRelayResident(int dt, int bm, int bn, int M, int N, int K, int rows_per_tile, int sk_wgs)
{
    if (sk_wgs > 0) return sk_wgs <= CuCount() * GemmWgsPerCu(dt, 256, 256, K, true);
    if (rows_per_tile <= 0 || rows_per_tile % bm != 0 || M % rows_per_tile != 0) return false;
    const int per = (rows_per_tile / bm) * ((N + bn - 1) / bn);
    return per <= CuCount() * GemmWgsPerCu(dt, bm, bn, K, false);
}

// Stream-K plan of a GEMM whose data-parallel tiling leaves CUs idle.
// Default: an exact split of K over 256x256 tiles, S = CUs / tiles pieces per
// tile, each piece at least 16 K stages (S >= 2), so every workgroup runs one
// piece and the workgroups of an XCD walk K in step on a compact patch of
// tiles; where the best data-parallel tiling fills less than 60% of the
// device's workgroup slots, or less than 90% with K of at least 256 stages
// (16384), where two long pieces per 256x256 tile amortise the fix-up. The
// last piece to finish sums all S partials alone, so short pieces lose to
// that fix-up. Measured on MI355X with a warm activation: 2048x896x4864
// data-parallel 67.1 us (best tile), 2 pieces 65.7, 4 pieces (19 stages)
// 53.6, 8 pieces (9.5 stages) 78.2; 2048x896x896 with 2 pieces of 7 stages
// 32.3 against 21.0. 2048x3584x18944 (the data-parallel 256x128 tiles fill
// 87.5%): 226 us in two pieces of 148 stages against 248 us data-parallel in
// the 7B prefill, on the 16x16x32 staged loop (KR_GEMM_SK_LONGK=0 keeps it
// data-parallel). Spreading the iterations of every tile over all 256 CUs
// instead (pieces of uneven length at different K offsets, sharing no
// operand lines) took 369 us for 2048x3584x18944. KR_GEMM_SK_WGS=G forces that
// even spread over G workgroups (a measurement aid).
bool PlanStreamK(int M, int N, int K, StreamKPlan &pl)
{
    if (K % kPipeK != 0 || M < 256 || N < 256) return false;
    pl.tiles = ((M + 255) / 256) * ((N + 255) / 256);
    pl.nk = K / kPipeK;
    if (const char *e = std::getenv("KR_GEMM_SK_WGS")) {
        pl.G = std::max(1, std::atoi(e));
        if (pl.tiles >= pl.G || int64_t(pl.tiles) * pl.nk < 4 * int64_t(pl.G)) return false;
    } else {
        const GemmTile dp = GemmPickTile(M, N, 0, false);
        const int dp_tiles = ((M + dp.bm - 1) / dp.bm) * ((N + dp.bn - 1) / dp.bn);
        const int dp_slots = CuCount() * (dp.bm * dp.bn >= 256 * 128 ? 1 : 2);
        const int dp_rounds = (dp_tiles + dp_slots - 1) / dp_slots;
        const double fill = double(dp_tiles) / (double(dp_rounds) * dp_slots);
        static const bool longk = [] {
            const char *e = std::getenv("KR_GEMM_SK_LONGK");
            return e == nullptr || std::atoi(e) != 0;
        }();
        static const int longk_nk = [] {
            const char *e = std::getenv("KR_GEMM_SK_LONGK_NK");
            return e != nullptr ? std::max(32, std::atoi(e)) : 256;
        }();
        if (fill >= 0.6 && !(longk && fill < 0.9 && pl.nk >= longk_nk)) return false;
        const int S = std::min(CuCount() / pl.tiles, pl.nk / 16);
        if (S < 2) return false;
        pl.G = S * pl.tiles;
    }
    const int64_t I = int64_t(pl.tiles) * pl.nk;
    if ((I + pl.G - 1) / pl.G > pl.nk) return false;  // a run spans at most two pieces
    auto owner = [&](int64_t x) { return int(((x + 1) * pl.G - 1) / I); };
    pl.pmax = 1;
    for (int t = 0; t < pl.tiles; ++t)
        pl.pmax = std::max(pl.pmax, owner(int64_t(t) * pl.nk + pl.nk - 1) - owner(int64_t(t) * pl.nk) + 1);
    return true;
}

template <int DT, int BM, int BN>
void LaunchTyped(const GemmParams &base, int order_rows, int tail_tiles, hipStream_t stream,
                 const StreamKPlan *sk = nullptr)
{
    GemmParams p = base;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    // relay order needs whole relay tiles of whole row blocks
    auto whole = [&](int rows) { return rows > 0 && rows % BM == 0 && p.tiles_m % (rows / BM) == 0; };
    p.order_rows = 0;
    if (p.pub.ctrl != nullptr && sk != nullptr) {
        // stream-K: each tile's finisher arrives once on every relay tile its
        // rows cover, so a relay tile waits for (row blocks in it) x tiles_n
        // arrivals, or tiles_n when it is shorter than a row block
        const int R = p.pub.rows_per_tile;
        if (R <= 0 || (R % BM != 0 && BM % R != 0) || p.M % R != 0)
            throw std::runtime_error("gemm: stream-K relay tiles must be whole row blocks or divide one");
        p.pub.arrivals = (R >= BM ? R / BM : 1) * p.tiles_n;
    } else if (p.pub.ctrl != nullptr) {
        if (!whole(p.pub.rows_per_tile)) throw std::runtime_error("relay tile rows must be a multiple of BM dividing M");
        p.pub.arrivals = (p.pub.rows_per_tile / BM) * p.tiles_n;
        p.order_rows = p.pub.rows_per_tile;
        if (order_rows > 0) {
            if (order_rows % p.pub.rows_per_tile != 0 || !whole(order_rows))
                throw std::runtime_error("gemm: order_rows must be a multiple of the relay tile dividing M");
            p.order_rows = order_rows;
        }
    } else if (p.wait.ctrl != nullptr && p.wait.row_off == 0 && whole(p.wait.prod_rows)) {
        p.order_rows = p.wait.prod_rows;  // the rows that are released first run first
    }
    p.gemm_wgs = p.tiles_m * p.tiles_n;
    p.group_m = RasterGroupM();
    if (p.rn_y != nullptr) {
        if (sk == nullptr && p.order_rows != p.pub.rows_per_tile)
            throw std::runtime_error("gemm: the Add+RMSNorm relay consumer needs the default relay-tile order");
        if (!NormRelayResident(DT, BM, BN, p.M, p.N, p.K, p.pub.rows_per_tile, sk != nullptr ? sk->G : 0))
            throw std::runtime_error("gemm: a relay tile's producer workgroups do not fit the device at once; "
                                     "the Add+RMSNorm relay consumer would wait on workgroups not yet placed");
        // a grid resident as a whole releases every tile at about the same
        // time whatever the order: keep the grouped raster (square patches
        // per XCD, less operand traffic than relay-tile order)
        if (sk == nullptr && p.gemm_wgs <= CuCount() * GemmWgsPerCu<DT, BM, BN>(p.K, false)) p.order_rows = 0;
    }
    if (sk != nullptr) {
        if (BM != 256 || BN != 256 || sk->tiles != p.gemm_wgs) throw std::logic_error("gemm: stream-K plan mismatch");
        p.sk_wgs = sk->G;
        p.sk_pmax = sk->pmax;
        p.gemm_wgs = sk->G;
    }
    int grid_x = p.gemm_wgs;
    if (p.tail_act != nullptr) {
        p.tail_wpt = 256;  // one per CU of the device: enough to fill the idle CUs of the last round
        grid_x += tail_tiles * p.tail_wpt;
    }
    const dim3 grid(grid_x);
    int threads = 0;
    const GemmFn fn = PickGemmKernel<DT, BM, BN>(p.K, sk != nullptr, threads);
    void *args[] = {&p};
    Check(hipLaunchKernel(reinterpret_cast<const void *>(fn), grid, dim3(threads), args, 0, stream), "gemm launch");
}

}  // namespace

namespace {

int Waves(int tiles, int slots) { return (tiles + slots - 1) / slots; }

}  // namespace

GemmTile GemmPickTile(int M, int N, int relay_rows, bool coresident)
{
    // Candidates from most to least data reuse; take the first that keeps the
    // device busy (>= 2 full waves of workgroups, or whole waves) or, failing
    // that, the one with the best wave efficiency. A GEMM whose 128x128 tiles
    // give every workgroup a CU of its own takes them: with so few workgroups
    // each CU's load path is the limit, and smaller tiles put more CUs to work
    // (MI355X, K 896: 2048x896 21.0 us against 24.0 for 128x256, 2048x1152
    // 20.6 against 23.8). Every tile runs the same MFMA and K order, so the
    // choice never changes the arithmetic.
    static const GemmTile cands[] = {{256, 256}, {256, 128}, {128, 256}, {128, 128}, {64, 256}};
    const int cus = 256;
    if ((relay_rows == 0 || relay_rows % 128 == 0) && ((M + 127) / 128) * ((N + 127) / 128) <= cus)
        return {128, 128};
    // share of the device's slots the tiles' useful work fills
    auto fill = [&](GemmTile t) {
        const int tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
        const int slots = cus * (t.bm * t.bn >= 256 * 128 ? 1 : 2);
        return double(M) * N / (double(Waves(tiles, slots)) * slots * t.bm * t.bn);
    };
    // 192x256 (three 32-row blocks per wave of the 8-wave grid) for a GEMM
    // that 256x256 tiles leave a third idle and no smaller tile fills better,
    // e.g. q/k/v 2048x4608: 198 tiles fill 75% against 144 tiles' 56%
    // (without relay releases, waits or co-residency)
    const bool try192 = relay_rows == 0 && !coresident;
    GemmTile best{-1, -1};
    double best_eff = -1.0;
    auto pick192 = [&](GemmTile other) {
        return try192 && fill({192, 256}) > 1.15 * fill(other) ? GemmTile{192, 256} : other;
    };
    for (const GemmTile &t : cands) {
        if (relay_rows > 0 && relay_rows % t.bm != 0) continue;
        if (coresident && t.bm * t.bn >= 256 * 256) continue;
        const int tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
        const int slots = cus * (t.bm * t.bn >= 256 * 128 ? 1 : 2);
        // enough workgroups for two rounds, or whole rounds exactly
        if (tiles >= 2 * slots || tiles % slots == 0) return t.bm == 256 && t.bn == 256 ? t : pick192(t);
        const double work = double(t.bm) * t.bn;  // per-workgroup work unit
        const double eff = double(tiles) * work / (double(Waves(tiles, slots)) * slots * work);
        const double score = eff * (t.bm * t.bn >= 256 * 128 ? 1.0 : 0.85);
        if (score > best_eff) {
            best_eff = score;
            best = t;
        }
    }
    return best.bm < 0 ? best : pick192(best);
}

bool GemmNormRelayFits(int M, int N, int K, int rows_per_tile, bool streamk_ws, int dtype)
{
    if (AddRmsNormRowCpl(N) == 0 || rows_per_tile <= 0 || M % rows_per_tile != 0) return false;
    StreamKPlan skp;
    const bool sk_pub_ok = rows_per_tile % 256 == 0 || 256 % rows_per_tile == 0;
    if (streamk_ws && sk_pub_ok && !ForceSimple() && PlanStreamK(M, N, K, skp))
        return NormRelayResident(dtype, 256, 256, M, N, K, rows_per_tile, skp.G);
    GemmTile t = GemmPickTile(M, N, rows_per_tile, false);
    if (const char *e = std::getenv("KR_GEMM_TILE")) {
        int bm = 0, bn = 0;
        if (std::sscanf(e, "%dx%d", &bm, &bn) == 2 && rows_per_tile % bm == 0) t = {bm, bn};
    }
    if (t.bm <= 0 || t.bm == 192) t = {256, 256};
    return NormRelayResident(dtype, t.bm, t.bn, M, N, K, rows_per_tile, 0);
}

void GemmStreamKNeeds(int M, int N, int K, size_t *ws_bytes, int *counters)
{
    StreamKPlan pl;
    if (PlanStreamK(M, N, K, pl)) {
        *ws_bytes = size_t(pl.tiles) * pl.pmax * 256 * 256 * 4;
        *counters = pl.tiles;
    } else {
        *ws_bytes = 0;
        *counters = 0;
    }
}

// Wave tail of a plain data-parallel 256x256 grid (the 8-wave staged kernel,
// no relay, no RoPE / norm / unary epilogue, no forced tile): when its tiles
// are not a whole number of rounds on the device, the last round runs partly
// idle (gate/up 2048x37888: 1184 tiles = 4 rounds + 160). Then the columns
// that fill whole rounds stay one launch (a), and the rest run as a second
// launch (b) of 192x256 tiles, one round of three-quarter tiles instead of a
// full round. Every tile shape runs the same MFMA over the same k16 chunks
// in the same order: the same bits. The SwiGLU epilogue splits with C (its
// gate/up groups of 8 never straddle a 256-column boundary).
// KR_GEMM_TAIL=0 keeps one launch.
bool SplitWaveTail(const GemmDesc &d, GemmDesc &a, GemmDesc &b)
{
    static const bool on = [] {
        const char *e = std::getenv("KR_GEMM_TAIL");
        return e == nullptr || std::atoi(e) != 0;
    }();
    if (!on || d.bm != 0 || d.bn != 0 || d.coresident || d.order_rows != 0) return false;
    if (d.pub.ctrl != nullptr || d.wait.ctrl != nullptr || d.tail_act != nullptr || d.y != nullptr ||
        d.rope_cos != nullptr || d.norm_y != nullptr)
        return false;
    if (d.K % kPipeK != 0 || ForceSimple() || MainLoopMode() != 2 || PipeWaves() != 8) return false;
    const GemmTile t = GemmPickTile(d.M, d.N, 0, false);
    if (t.bm != 256 || t.bn != 256) return false;
    StreamKPlan skp;
    if (d.streamk && PlanStreamK(d.M, d.N, d.K, skp)) return false;
    const int64_t cus = CuCount();
    const int64_t tm = (d.M + 255) / 256, tn = (d.N + 255) / 256;
    const int64_t rounds = tm * tn / cus;
    if (rounds < 1 || (tm * tn) % cus == 0 || (rounds * cus) % tm != 0) return false;
    const int64_t n1 = rounds * cus / tm * 256;  // columns of the whole rounds
    const int64_t n2 = d.N - n1;
    if (n2 <= 0 || ((d.M + 191) / 192) * ((n2 + 255) / 256) > cus) return false;
    a = d;
    b = d;
    a.N = int(n1);
    a.bm = 256;
    a.bn = 256;
    b.N = int(n2);
    b.bm = 192;
    b.bn = 256;
    b.Bt = static_cast<const uint16_t *>(d.Bt) + n1 * d.ldb;
    if (d.C != nullptr) b.C = static_cast<uint16_t *>(d.C) + n1;
    if (d.bias != nullptr) b.bias = static_cast<const uint16_t *>(d.bias) + n1;
    if (d.epi_act != nullptr) b.epi_act = static_cast<uint16_t *>(d.epi_act) + n1 / 2;
    return true;
}

void GemmLaunch(const GemmDesc &d, hipStream_t stream)
{
    if (d.K % 8 != 0) throw std::runtime_error("gemm: K must be a multiple of 8");
    if (d.M <= 0 || d.N <= 0 || d.K <= 0) throw std::runtime_error("gemm: empty shape");
    if ((reinterpret_cast<uintptr_t>(d.A) | reinterpret_cast<uintptr_t>(d.Bt)) & 15)
        throw std::runtime_error("gemm: A/Bt must be 16-byte aligned");
    if ((d.lda | d.ldb) % 8 != 0) throw std::runtime_error("gemm: lda/ldb must be multiples of 8");
    {
        GemmDesc a, b;
        if (SplitWaveTail(d, a, b)) {
            GemmLaunch(a, stream);
            GemmLaunch(b, stream);
            return;
        }
    }
    GemmParams p{};
    p.A = static_cast<const uint16_t *>(d.A);
    p.Bt = static_cast<const uint16_t *>(d.Bt);
    p.C = static_cast<uint16_t *>(d.C);
    p.bias = static_cast<const uint16_t *>(d.bias);
    p.lda = d.lda;
    p.ldb = d.ldb;
    p.ldc = d.ldc;
    p.M = d.M;
    p.N = d.N;
    p.K = d.K;
    p.pub = d.pub;
    p.wait = d.wait;
    p.store_kind = StoreKind();
    p.tail_act = static_cast<uint16_t *>(d.tail_act);
    p.tail_cols = d.tail_cols;
    p.epi_act = static_cast<uint16_t *>(d.epi_act);
    p.ld_act = d.ld_act;
    p.uy = d.y;
    p.uop = d.y_op;
    p.udt = d.y_dtype;
    p.ldy = d.ld_y > 0 ? d.ld_y : d.N;
    if (d.y != nullptr) {
        if (d.y_op != kEwGelu && d.y_op != kEwSilu && d.y_op != kEwCast)
            throw std::runtime_error("gemm: the unary consumer must be gelu, silu or cast");
        if (d.y_dtype != kBF16 && d.y_dtype != kF16 && d.y_dtype != kF32)
            throw std::runtime_error("gemm: unary consumer dtype");
        if (d.epi_act != nullptr || d.tail_act != nullptr || d.norm_y != nullptr || d.rope_cos != nullptr)
            throw std::runtime_error("gemm: one epilogue consumer per launch");
        if ((reinterpret_cast<uintptr_t>(d.y) & 15) != 0 || (p.ldy * int64_t(DTypeBytes(d.y_dtype))) % 16 != 0)
            throw std::runtime_error("gemm: unary consumer output must be 16-byte aligned rows");
    }
    if (d.rope_cos != nullptr) {
        if (d.rope_sin == nullptr || (d.rope_d != 64 && d.rope_d != 128) || d.rope_cols <= 0 ||
            d.rope_cols % d.rope_d != 0 || d.rope_cols > d.N || d.rope_pos0 < 0)
            throw std::runtime_error("gemm: RoPE epilogue needs cos/sin tables, head size 64 or 128, whole heads");
        if (p.epi_act != nullptr) throw std::runtime_error("gemm: RoPE and SwiGLU epilogues are exclusive");
        if ((reinterpret_cast<uintptr_t>(d.rope_cos) | reinterpret_cast<uintptr_t>(d.rope_sin)) & 15)
            throw std::runtime_error("gemm: RoPE tables must be 16-byte aligned");
        // every tile width is a multiple of 128, so tiles start on head boundaries
        p.rope_cos = static_cast<const uint16_t *>(d.rope_cos);
        p.rope_sin = static_cast<const uint16_t *>(d.rope_sin);
        p.rope_cols = d.rope_cols;
        p.rope_d = d.rope_d;
        p.rope_pos0 = d.rope_pos0;
    }
    if (p.epi_act != nullptr) {
        if (p.tail_act != nullptr) throw std::runtime_error("gemm: SwiGLU epilogue and tail consumer are exclusive");
        if (d.dtype != kBF16 && d.dtype != kF16) throw std::runtime_error("gemm swiglu: 16-bit output only");
        if (d.N % 16 != 0) throw std::runtime_error("gemm swiglu: N must be a multiple of 16 (gate/up groups of 8)");
        if ((reinterpret_cast<uintptr_t>(d.epi_act) & 15) || d.ld_act % 8 != 0 || d.ld_act < d.N / 2)
            throw std::runtime_error("gemm swiglu: act must be 16-byte aligned with ld_act >= N/2, a multiple of 8");
    }
    if (p.tail_act != nullptr) {
        if (p.pub.ctrl == nullptr || d.M % p.pub.rows_per_tile != 0)
            throw std::runtime_error("gemm tail: needs a relay release over whole tiles of M");
        if (d.dtype != kBF16 && d.dtype != kF16) throw std::runtime_error("gemm tail: 16-bit output only");
        if (d.N != 2 * d.tail_cols || d.ldc != d.N || d.tail_cols % 8 != 0)
            throw std::runtime_error("gemm tail: C must be a packed [M, 2*cols] interleaved gate/up buffer");
        if ((reinterpret_cast<uintptr_t>(d.C) | reinterpret_cast<uintptr_t>(d.tail_act)) & 15)
            throw std::runtime_error("gemm tail: buffers must be 16-byte aligned");
    }
    if (d.norm_y != nullptr) {
        if (d.pub.ctrl == nullptr || d.pub.rows_per_tile <= 0 || d.M % d.pub.rows_per_tile != 0)
            throw std::runtime_error("gemm add_rmsnorm: needs a relay release over whole tiles of M");
        if (d.norm_res == nullptr || d.norm_gamma == nullptr)
            throw std::runtime_error("gemm add_rmsnorm: residual and gamma are required");
        if (p.epi_act != nullptr || p.tail_act != nullptr || d.rope_cos != nullptr || d.order_rows != 0)
            throw std::runtime_error("gemm add_rmsnorm: excludes the SwiGLU epilogue/tail, RoPE and order_rows");
        if (d.ldc != d.N || AddRmsNormRowCpl(d.N) == 0)
            throw std::runtime_error("gemm add_rmsnorm: C must be packed (ldc == N) with N in 136..4096, N % 8 == 0");
        if ((reinterpret_cast<uintptr_t>(d.C) | reinterpret_cast<uintptr_t>(d.norm_res) |
             reinterpret_cast<uintptr_t>(d.norm_gamma) | reinterpret_cast<uintptr_t>(d.norm_y) |
             reinterpret_cast<uintptr_t>(d.norm_sum)) & 15)
            throw std::runtime_error("gemm add_rmsnorm: buffers must be 16-byte aligned");
        p.rn_res = static_cast<const uint16_t *>(d.norm_res);
        p.rn_gamma = static_cast<const uint16_t *>(d.norm_gamma);
        p.rn_y = static_cast<uint16_t *>(d.norm_y);
        p.rn_sum = static_cast<uint16_t *>(d.norm_sum);
        p.rn_rstd = d.norm_rstd;
        p.rn_eps = d.norm_eps;
        p.rn_cpl = AddRmsNormRowCpl(d.N);
        p.rn_spins = d.norm_max_spins > 0 ? d.norm_max_spins : kDefaultMaxSpins;
    }
    if (p.wait.ctrl != nullptr && p.wait.prod_rows <= 0) throw std::runtime_error("gemm: wait.prod_rows must be > 0");
    const int relay_rows = d.pub.ctrl != nullptr ? d.pub.rows_per_tile : 0;
    GemmTile t = GemmPickTile(d.M, d.N, relay_rows, d.coresident);
    if (const char *e = std::getenv("KR_GEMM_TILE")) {
        // tile sweep override "BMxBN" (measurement aid; bits are unchanged)
        int bm = 0, bn = 0;
        if (std::sscanf(e, "%dx%d", &bm, &bn) == 2 && (relay_rows == 0 || relay_rows % bm == 0)) t = {bm, bn};
    }
    if (d.bm > 0) {
        // a forced M tile pairs with the widest N tile built for it
        t.bm = d.bm;
        t.bn = d.bn > 0 ? d.bn : 256;
    } else if (d.bn > 0) {
        t.bn = d.bn;
    }
    if (t.bm < 0) throw std::runtime_error("gemm: relay tile rows must be a multiple of 64");
    if (d.epi_act != nullptr && t.bn < 256) t = {t.bm >= 256 ? 256 : 128, 256};  // the epilogue pairs 16-col groups
    // 192x256 runs only on the staged 8-wave kernel; elsewhere 256x256 (the
    // same MFMA and K order: the same bits)
    if (t.bm == 192 && (d.K % kPipeK != 0 || ForceSimple() || MainLoopMode() != 2 ||
                        d.tail_act != nullptr || d.pub.ctrl != nullptr || d.wait.ctrl != nullptr))
        t = {256, 256};
    const bool bf = d.dtype == kBF16;
    if (d.dtype != kBF16 && d.dtype != kF16) throw std::runtime_error("gemm: dtype must be bf16 or f16");
    const int order = d.order_rows;
    int tail = 0;
    if (d.tail_act != nullptr) {
        const int k = d.M / d.pub.rows_per_tile;
        tail = d.tail_tiles > 0 ? std::min(d.tail_tiles, k) : k;
    }
    StreamKPlan skp;
    // (a publishing split needs relay tiles that are whole 256-row blocks or
    // divide one)
    const int rpt = d.pub.rows_per_tile;
    const bool sk_pub_ok =
        d.pub.ctrl == nullptr || (rpt > 0 && (rpt % 256 == 0 || 256 % rpt == 0) && d.M % rpt == 0);
    if (d.streamk && sk_pub_ok && d.wait.ctrl == nullptr && d.tail_act == nullptr && d.epi_act == nullptr && !ForceSimple() &&
        d.bm == 0 && d.bn == 0 && PlanStreamK(d.M, d.N, d.K, skp) && d.sk_ws != nullptr && d.sk_cnt != nullptr &&
        d.sk_ws_bytes >= size_t(skp.tiles) * skp.pmax * 256 * 256 * 4 && d.sk_cnt_len >= skp.tiles &&
        (d.norm_y == nullptr || skp.G <= CuCount())) {
        p.sk_ws = static_cast<float *>(d.sk_ws);
        p.sk_cnt = d.sk_cnt;
        bf ? LaunchTyped<kBF16, 256, 256>(p, 0, 0, stream, &skp) : LaunchTyped<kF16, 256, 256>(p, 0, 0, stream, &skp);
        return;
    }
#define KR_GEMM_CASE(BM_, BN_)                                                                     \
    if (t.bm == BM_ && t.bn == BN_) {                                                              \
        bf ? LaunchTyped<kBF16, BM_, BN_>(p, order, tail, stream)                                  \
           : LaunchTyped<kF16, BM_, BN_>(p, order, tail, stream);                                  \
        return;                                                                                    \
    }
    KR_GEMM_CASE(256, 256)
    KR_GEMM_CASE(192, 256)
    KR_GEMM_CASE(256, 128)
    KR_GEMM_CASE(128, 256)
    KR_GEMM_CASE(128, 128)
    KR_GEMM_CASE(64, 256)
#undef KR_GEMM_CASE
    throw std::runtime_error("gemm: unsupported tile " + std::to_string(t.bm) + "x" + std::to_string(t.bn));
}

}  // namespace kr
