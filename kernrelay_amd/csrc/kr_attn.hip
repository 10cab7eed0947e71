// Causal GQA flash attention on CDNA4 MFMA (BSND layout).
//
// Replaces the reference's aclnnFlashAttentionScore call (FlashN,
// exec/qwen_main.cpp:591-614: scale 1/sqrt(D), keepProb 1, sparseMode 3 with
// the upper-triangular mask of MakeMask :487-497).
//
// One workgroup = 128 queries of one head (4 waves x 32 queries); keys and
// values stream through a double-buffered LDS ring in blocks of 64: block
// kb+1 is loaded into registers while block kb is computed, then written to
// the other buffer, one barrier per block. The kernel computes the
// transposed products so that every operand lands where the next MFMA wants
// it, with no cross-lane shuffles of P:
//   S^T = K . Q^T   (32x32x16: A = K rows from LDS, B = Q rows in registers)
//       -> lane l holds query l%32 and 16 keys of each 32-key half; the row
//          max / sum over keys is a lane-local loop plus one xor-32 shuffle.
//   O^T += V^T . P^T (A = V^T from a transposed LDS copy, B = P^T straight
//          from the S^T accumulators after rounding to 16 bits).
// MFMA pairs A slot s with B slot s, so the key order inside a 16-key step
// only has to agree between V^T and P^T. P^T's order is the accumulator's
// {4h..4h+3, 8+4h..8+4h+3} for lane half h; V^T rows are stored with the keys
// of each 16-key group permuted into exactly that order, so one ds_read_b128
// fetches a lane's 8 keys.
// Online softmax in base 2 (exponent fma(score, scale*log2(e), -m)), fp32
// state, with the running max m moved lazily (see the loop).
// Workgroups run heaviest (longest causal rows) first across all heads.
#include <algorithm>
#include <vector>

#include "kr_misc.h"

namespace kr {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kKvBlk = 64;
typedef uint32_t AttnU32x4 __attribute__((ext_vector_type(4)));

// two values to 16 bits (round to nearest even, as Elem<DT>::Store), packed
// low | high << 16: one v_cvt_pk_bf16_f32 for bf16
template <int DT>
__device__ __forceinline__ uint32_t Pack2(float lo, float hi)
{
    if constexpr (DT == kBF16) {
        typedef float F2 __attribute__((ext_vector_type(2)));
        typedef __bf16 B2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((F2){lo, hi}, B2));
    } else {
        return uint32_t(Elem<DT>::Store(lo)) | (uint32_t(Elem<DT>::Store(hi)) << 16);
    }
}
constexpr int kQBlk = 128;

// Work items, heaviest first: workgroup b runs item b / HQ of head b % HQ.
// An item is query block qb over key blocks [kb_lo, kb_hi); a query block
// whose causal row is long is cut into `pieces` items (split id sid), each
// writing its fp32 partial (O, m, l); the last piece to finish sums them in
// piece order.
constexpr int kMaxItems = 128;
struct AttnItem {
    int16_t qb, kb_lo, kb_hi, piece, pieces, sid;
};

struct AttnParams {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    uint16_t *o;
    int64_t ldq, ldk, ldv, ldo;  // row strides (elements) of the [S, heads*D] views
    int S, HQ, HKV;
    float scale_log2;
    float *ws;       // split partials [sid][HQ][pmax][chunks][256 threads][4]
    int32_t *cnt;    // [sid][HQ] arrival tickets, zero between launches
    int pmax;
    AttnItem items[kMaxItems];
};

template <int DT>
__device__ __forceinline__ f32x16 Mfma(const uint4 &a, const uint4 &b, const f32x16 &c)
{
    if constexpr (DT == kBF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

template <int D>
__device__ __forceinline__ int KSwz(int r, int c)
{
    if constexpr (D == 128) return c ^ (r & 15);
    else return c ^ ((r >> 1) & 7);
}

// V^T rows hold 64 keys = 8 chunks of 16 bytes; chunk c of row d sits in
// slot c ^ VSwz(d) (distinct slots for 8- and 16-lane passes).
__device__ __forceinline__ int VSwz(int d) { return (d & 7) ^ ((d >> 3) & 1); }

template <int DT, int D>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2))) AttnKernel(AttnParams p)
{
    constexpr int DCH = D / 8;                       // 16-byte chunks per K/V row
    constexpr int DBLK = D / 32;
    constexpr int KL = kKvBlk * DCH / 256;           // K chunks per thread per block
    constexpr int VG = (kKvBlk / 4) * DCH;           // V (4 keys x 8 d) groups per block
    constexpr int VL = (VG + 255) / 256;             // V groups per thread
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kKvBlk * D];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * kKvBlk];

    __shared__ int last_piece;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hf = lane >> 5;
    const int h = int(blockIdx.x) % p.HQ;
    const AttnItem item = p.items[int(blockIdx.x) / p.HQ];
    const int qb = item.qb;
    const int q0 = qb * kQBlk;
    const int kvh = h / (p.HQ / p.HKV);
    const int64_t ldq = p.ldq;
    const int qrow = q0 + wave * 32 + (lane & 31);
    const int wave_q_hi = min(q0 + wave * 32 + 31, p.S - 1);

    uint4 qf[D / 16];
#pragma unroll
    for (int dc = 0; dc < D / 16; ++dc) {
        if (qrow < p.S) {
            qf[dc] = *reinterpret_cast<const uint4 *>(p.q + int64_t(qrow) * ldq + int64_t(h) * D + dc * 16 + hf * 8);
        } else {
            qf[dc] = make_uint4(0, 0, 0, 0);
        }
    }

    f32x16 oacc[DBLK];
#pragma unroll
    for (int b = 0; b < DBLK; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[b][v] = 0.0f;
    float m = -INFINITY;
    float l = 0.0f;

    const int kb_lo = item.kb_lo, kb_hi = item.kb_hi;

    // block kb -> registers, with no branch around a load: rows past S read
    // row S-1 again (their keys are masked to -inf, so their P is exactly 0
    // and their finite K and V rows contribute nothing), threads past the
    // block's V groups (D 64) read group 0 again and never store it. Plain
    // vector types: struct copies would go through memcpy, which keeps the
    // arrays in scratch memory.
    AttnU32x4 kr[KL];
    AttnU32x4 vr[VL][4];
    // this thread's element offsets inside a block of K / V rows
    int koff[KL], voff[VL][4];
#pragma unroll
    for (int i = 0; i < KL; ++i) {
        const int t = tid + 256 * i;
        koff[i] = (t / DCH) * int(p.ldk) + kvh * D + (t % DCH) * 8;
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
        const int t = tid + 256 * i;
        const int grp = t < VG ? t / DCH : 0, c = t % DCH;
#pragma unroll
        for (int r = 0; r < 4; ++r) voff[i][r] = (4 * grp + r) * int(p.ldv) + kvh * D + c * 8;
    }
    auto load = [&](int kb) {
        const int kv0 = kb * kKvBlk;
        if (kv0 + kKvBlk <= p.S) {
            // a whole block inside S: the block's base plus this thread's offsets
            const uint16_t *kbase = p.k + int64_t(kv0) * p.ldk;
            const uint16_t *vbase = p.v + int64_t(kv0) * p.ldv;
#pragma unroll
            for (int i = 0; i < KL; ++i) kr[i] = *reinterpret_cast<const AttnU32x4 *>(kbase + koff[i]);
#pragma unroll
            for (int i = 0; i < VL; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) vr[i][r] = *reinterpret_cast<const AttnU32x4 *>(vbase + voff[i][r]);
            return;
        }
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const int t = tid + 256 * i;
            const int kv = min(kv0 + t / DCH, p.S - 1);
            kr[i] = *reinterpret_cast<const AttnU32x4 *>(p.k + int64_t(kv) * p.ldk + int64_t(kvh) * D + (t % DCH) * 8);
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const int t = tid + 256 * i;
            const int grp = t < VG ? t / DCH : 0, c = t % DCH;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kv = min(kv0 + 4 * grp + r, p.S - 1);
                vr[i][r] = *reinterpret_cast<const AttnU32x4 *>(p.v + int64_t(kv) * p.ldv + int64_t(kvh) * D + c * 8);
            }
        }
    };
    // registers -> LDS buffer b: K row-major (swizzled), V transposed with
    // each 16-key group permuted to the P^T slot order
    auto store = [&](int b) {
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            const int t = tid + 256 * i;
            const int r = t / DCH, c = t % DCH;
            *reinterpret_cast<AttnU32x4 *>(&Ks[b][r * D + KSwz<D>(r, c) * 8]) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) {
            const int t = tid + 256 * i;
            if (VG % 256 != 0 && t >= VG) continue;  // (D 64: half the threads)
            const int ap = t / DCH, c = t % DCH;  // keys 4ap..4ap+3, d chunk c
            const int u = 4 * (ap >> 2) + ((ap & 3) >> 1) + 2 * (ap & 1);  // 8-byte unit in the row
            const AttnU32x4 &w0 = vr[i][0], &w1 = vr[i][1], &w2 = vr[i][2], &w3 = vr[i][3];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = c * 8 + e;
                // the 16-bit halves e&1 of keys (0, 1) and (2, 3), paired by
                // one byte permute each: v_perm_b32(hi, lo, sel) picks bytes
                // of the 64-bit {hi, lo}, sel 0x05040100 = low halves,
                // 0x07060302 = high halves
                const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
                *reinterpret_cast<uint2 *>(&Vt[b][d * kKvBlk + (((u >> 1) ^ VSwz(d)) * 8) + (u & 1) * 4]) =
                    make_uint2(__builtin_amdgcn_perm(w1[e >> 1], w0[e >> 1], sel),
                               __builtin_amdgcn_perm(w3[e >> 1], w2[e >> 1], sel));
            }
        }
    };

    load(kb_lo);
    store(0);
    __syncthreads();

    for (int kb = kb_lo; kb < kb_hi; ++kb) {
        const int kv0 = kb * kKvBlk;
        const int cur = (kb - kb_lo) & 1;
        const bool more = kb + 1 < kb_hi;
        if (more) load(kb + 1);

        if (kv0 <= wave_q_hi) {  // else: block entirely in this wave's future
            const uint16_t *K = Ks[cur];
            const uint16_t *V = Vt[cur];
            f32x16 sacc[2];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
                for (int v = 0; v < 16; ++v) sacc[kh][v] = 0.0f;
                const int r = kh * 32 + (lane & 31);
#pragma unroll
                for (int dc = 0; dc < D / 16; ++dc) {
                    const uint4 kf = *reinterpret_cast<const uint4 *>(K + r * D + KSwz<D>(r, dc * 2 + hf) * 8);
                    sacc[kh] = Mfma<DT>(kf, qf[dc], sacc[kh]);
                }
            }

            // raw scores: the row max is taken before scaling (scale > 0);
            // masked keys (above the diagonal, past S) by select, not branch
            float mloc = -INFINITY;
            const bool diag = kv0 + kKvBlk - 1 > q0 + wave * 32 || kv0 + kKvBlk > p.S;
            if (diag) {
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int kv = kv0 + kh * 32 + 8 * (v >> 2) + 4 * hf + (v & 3);
                        sacc[kh][v] = kv > qrow || kv >= p.S ? -INFINITY : sacc[kh][v];
                    }
            }
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int v = 0; v < 16; ++v) mloc = fmaxf(mloc, sacc[kh][v]);
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64)) * p.scale_log2;
            // lazy rescale: the row's reference max m moves only when a score
            // exceeds it by more than 2^8 (so p = 2^(s - m) <= 256, exact in
            // range for bf16 P and fp32 sums); the wave skips the O rescale
            // when no row moved. O / l is unchanged: both carry the same m.
            const bool move = mloc > m + 8.0f;
            const float mnew = move ? mloc : m;
            const float msub = mnew == -INFINITY ? 0.0f : mnew;
            const float alpha = move ? __builtin_amdgcn_exp2f(m - msub) : 1.0f;
            float lsum = 0.0f;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kh][v], p.scale_log2, -msub));
                    sacc[kh][v] = pv;
                    lsum += pv;
                }
            l = l * alpha + lsum;
            m = mnew;
            if (__builtin_expect((__builtin_amdgcn_read_exec() & __ballot(move)) != 0, 0)) {
#pragma unroll
                for (int b = 0; b < DBLK; ++b)
#pragma unroll
                    for (int v = 0; v < 16; ++v) oacc[b][v] *= alpha;
            }

#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int kh = c >> 1;
                const int vb = (c & 1) * 8;
                uint32_t pw[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) pw[s] = Pack2<DT>(sacc[kh][vb + 2 * s], sacc[kh][vb + 2 * s + 1]);
                const uint4 pf = make_uint4(pw[0], pw[1], pw[2], pw[3]);
#pragma unroll
                for (int b = 0; b < DBLK; ++b) {
                    const int d = b * 32 + (lane & 31);
                    const uint4 vf = *reinterpret_cast<const uint4 *>(V + d * kKvBlk + (((2 * c + hf) ^ VSwz(d)) * 8));
                    oacc[b] = Mfma<DT>(vf, pf, oacc[b]);
                }
            }
        }
        if (more) store(cur ^ 1);  // the other buffer was last read before the previous barrier
        __syncthreads();
    }

    if (item.pieces > 1) {
        // split row: every piece writes its partial (agent-scope stores,
        // read back on any XCD); the last to arrive sums all of them in piece
        // order, so the result does not depend on which piece finishes last
        constexpr int NCH = DBLK * 4 + 1;  // 16-byte chunks per thread: O, then (m, l)
        const int64_t slot0 = (int64_t(item.sid) * p.HQ + h) * p.pmax;
        auto part = [&](int piece, int ch, int e) {
            return p.ws + (((slot0 + piece) * NCH + ch) * 256 + tid) * 4 + e;
        };
#pragma unroll
        for (int b = 0; b < DBLK; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                __hip_atomic_store(part(item.piece, b * 4 + v / 4, v % 4), oacc[b][v], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part(item.piece, NCH - 1, 0), m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part(item.piece, NCH - 1, 1), l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial is written
        __syncthreads();
        if (tid == 0) {
            int32_t *c = p.cnt + int64_t(item.sid) * p.HQ + h;
            const int32_t t = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_piece = t == item.pieces - 1;
            if (last_piece) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last_piece) return;
        float mp[4], lp[4];
        float mall = -INFINITY;
        for (int q = 0; q < item.pieces; ++q) {
            mp[q] = __hip_atomic_load(part(q, NCH - 1, 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lp[q] = __hip_atomic_load(part(q, NCH - 1, 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            mall = fmaxf(mall, mp[q]);
        }
        const float msub = mall == -INFINITY ? 0.0f : mall;
#pragma unroll
        for (int b = 0; b < DBLK; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[b][v] = 0.0f;
        l = 0.0f;
        for (int q = 0; q < item.pieces; ++q) {
            const float a = __builtin_amdgcn_exp2f(mp[q] - msub);  // 0 for an empty piece (m = -inf)
            l = __builtin_fmaf(lp[q], a, l);
#pragma unroll
            for (int b = 0; b < DBLK; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    oacc[b][v] = __builtin_fmaf(
                        __hip_atomic_load(part(q, b * 4 + v / 4, v % 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), a,
                        oacc[b][v]);
        }
    }
    l += __shfl_xor(l, 32, 64);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (qrow < p.S) {
        uint16_t *orow = p.o + int64_t(qrow) * p.ldo + int64_t(h) * D;
#pragma unroll
        for (int b = 0; b < DBLK; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = b * 32 + 8 * g + 4 * hf;
                uint2 w;
                w.x = uint32_t(Elem<DT>::Store(oacc[b][4 * g + 0] * inv)) |
                      (uint32_t(Elem<DT>::Store(oacc[b][4 * g + 1] * inv)) << 16);
                w.y = uint32_t(Elem<DT>::Store(oacc[b][4 * g + 2] * inv)) |
                      (uint32_t(Elem<DT>::Store(oacc[b][4 * g + 3] * inv)) << 16);
                *reinterpret_cast<uint2 *>(orow + d0) = w;
            }
    }
}

}  // namespace

namespace {

// Split plan: query block qb covers key blocks [0, nkb(qb)); rows longer than
// `cap` key blocks are cut into ceil(nkb / cap) pieces (at most 4), so no
// workgroup carries far more than the average and the grid's critical path
// shrinks. Items are ordered heaviest first.
struct AttnPlan {
    std::vector<AttnItem> items;
    int nsplit = 0, pmax = 1;
};

int AttnCap()
{
    static const int v = [] {
        const char *e = std::getenv("KR_ATTN_CAP");
        return e != nullptr ? std::max(1, std::atoi(e)) : 16;
    }();
    return v;
}

AttnPlan PlanAttn(int S, bool split)
{
    AttnPlan pl;
    const int nqb = (S + kQBlk - 1) / kQBlk;
    for (int qb = 0; qb < nqb; ++qb) {
        const int q_hi = std::min(qb * kQBlk + kQBlk - 1, S - 1);
        const int nkb = q_hi / kKvBlk + 1;
        const int pieces = split ? std::min(4, (nkb + AttnCap() - 1) / AttnCap()) : 1;
        const int sid = pieces > 1 ? pl.nsplit++ : 0;
        pl.pmax = std::max(pl.pmax, pieces);
        for (int pc = 0; pc < pieces; ++pc)
            pl.items.push_back({int16_t(qb), int16_t(nkb * pc / pieces), int16_t(nkb * (pc + 1) / pieces), int16_t(pc),
                                int16_t(pieces), int16_t(sid)});
    }
    std::stable_sort(pl.items.begin(), pl.items.end(), [](const AttnItem &a, const AttnItem &b) {
        const int wa = a.kb_hi - a.kb_lo, wb = b.kb_hi - b.kb_lo;
        return wa != wb ? wa > wb : a.qb > b.qb;
    });
    return pl;
}

}  // namespace

// Resident workgroup slots of the device (two 256-thread workgroups per CU).
int AttnSlots()
{
    static const int v = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return 2 * std::max(n, 1);
    }();
    return v;
}

void AttnSplitNeeds(int S, int HQ, int D, size_t *ws_bytes, int *counters)
{
    *ws_bytes = 0;
    *counters = 0;
    if (S <= 0 || HQ <= 0 || (D != 64 && D != 128)) return;
    // Split only a grid that leaves half the resident slots empty: a fuller
    // grid is bound by the CUs' MFMA, softmax and LDS throughput, not by its
    // longest row (measured on MI355X: 28 heads at S=2048 94 -> 116 us split,
    // 14 heads 59 -> 49 us).
    if (int64_t((S + kQBlk - 1) / kQBlk) * HQ * 2 > AttnSlots()) return;
    const AttnPlan pl = PlanAttn(S, true);
    if (pl.nsplit == 0 || pl.items.size() > size_t(kMaxItems)) return;
    *ws_bytes = size_t(pl.nsplit) * HQ * pl.pmax * (D / 32 * 4 + 1) * 256 * 16;
    *counters = pl.nsplit * HQ;
}

void AttnLaunch(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                void *out, int64_t ldo, int S, int HQ, int HKV, int D, float scale, hipStream_t stream,
                const AttnSplit *split)
{
    if (S <= 0) return;
    if (HQ <= 0 || HKV <= 0 || HQ % HKV != 0) throw std::runtime_error("attention: HQ must be a multiple of HKV");
    for (const void *ptr : {q, k, v, static_cast<const void *>(out)})
        if (reinterpret_cast<uintptr_t>(ptr) & 15) throw std::runtime_error("attention: pointers must be 16-byte aligned");
    AttnParams p{};
    p.q = static_cast<const uint16_t *>(q);
    p.k = static_cast<const uint16_t *>(k);
    p.v = static_cast<const uint16_t *>(v);
    p.o = static_cast<uint16_t *>(out);
    p.ldq = ldq > 0 ? ldq : int64_t(HQ) * D;
    p.ldk = ldk > 0 ? ldk : int64_t(HKV) * D;
    p.ldv = ldv > 0 ? ldv : int64_t(HKV) * D;
    p.ldo = ldo > 0 ? ldo : int64_t(HQ) * D;
    if ((p.ldq | p.ldk | p.ldv | p.ldo) % 8 != 0) throw std::runtime_error("attention: row strides must be multiples of 8");
    // the kernel addresses K/V rows inside a 64-row block by 32-bit offsets
    if (int64_t(std::max(p.ldk, p.ldv)) * 64 + int64_t(HKV) * D >= (int64_t(1) << 31))
        throw std::runtime_error("attention: K/V row strides too large");
    p.S = S;
    p.HQ = HQ;
    p.HKV = HKV;
    p.scale_log2 = scale * 1.4426950408889634f;
    // split rows only with a workspace that holds the plan's partials
    size_t need = 0;
    int ncnt = 0;
    if (split != nullptr) AttnSplitNeeds(S, HQ, D, &need, &ncnt);
    const bool use_split = split != nullptr && need > 0 && split->ws != nullptr && split->cnt != nullptr &&
                           split->ws_bytes >= need && split->cnt_len >= ncnt;
    const AttnPlan pl = PlanAttn(S, use_split);
    if (pl.items.size() > size_t(kMaxItems)) throw std::runtime_error("attention: sequence too long for the item table");
    std::copy(pl.items.begin(), pl.items.end(), p.items);
    p.ws = use_split ? split->ws : nullptr;
    p.cnt = use_split ? split->cnt : nullptr;
    p.pmax = pl.pmax;
    const dim3 grid(unsigned(pl.items.size()) * unsigned(HQ));
    const bool bf = dtype == kBF16;
    if (dtype != kBF16 && dtype != kF16) throw std::runtime_error("attention: dtype must be bf16 or f16");
    if (D == 128) {
        if (bf) hipLaunchKernelGGL((AttnKernel<kBF16, 128>), grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((AttnKernel<kF16, 128>), grid, dim3(256), 0, stream, p);
    } else if (D == 64) {
        if (bf) hipLaunchKernelGGL((AttnKernel<kBF16, 64>), grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((AttnKernel<kF16, 64>), grid, dim3(256), 0, stream, p);
    } else {
        throw std::runtime_error("attention: head_dim must be 64 or 128");
    }
    Check(hipGetLastError(), "attention launch");
}

}  // namespace kr
