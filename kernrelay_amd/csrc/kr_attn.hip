// Causal GQA flash attention on CDNA4 MFMA (BSND layout).
//
// Replaces the reference's aclnnFlashAttentionScore call (FlashN,
// exec/qwen_main.cpp:591-614: scale 1/sqrt(D), keepProb 1, sparseMode 3 with
// the upper-triangular mask of MakeMask :487-497).
//
// One workgroup = 128 queries of one head (4 waves x 32 queries) times KH
// key halves: with KH = 2 the workgroup has 8 waves, and waves 4..7 take the
// odd 64-key blocks of the same 128 queries while waves 0..3 take the even
// ones, merging their (m, l, O) through LDS at the end; that halves the
// longest causal row's walk, the critical path of a causal grid.
//
// Keys and values go global -> LDS by the direct-to-LDS DMA (kr_dma.h), both
// row-major, into a two-stage ring: stage s+1 is fetched while stage s is
// computed, one wait + barrier per stage, no VGPR staging. The 16-byte
// chunks of each row are XOR-swizzled on the source side (each DMA lane
// picks the chunk its LDS slot holds) so that the fragment reads below hit
// distinct banks.
//
// Products, chosen so that every operand lands where the next MFMA wants it:
//   S^T = K . Q^T   (v_mfma_f32_32x32x16: A = K rows by ds_read_b128, B = Q
//       rows held in registers) -> lane l holds query l % 32 and 16 keys of
//       each 32-key half; the row max / sum is a lane-local loop plus one
//       xor-32 shuffle.
//   O^T += V^T . P^T (A = V^T by ds_read_b64_tr_b16 from the row-major V,
//       B = P^T straight from the S^T accumulators rounded to 16 bits).
// ds_read_b64_tr_b16 hands lane 4a+b of each 16-lane group element b of the
// 8-byte pieces addressed by lanes a, a+4, a+8, a+12; when lane s addresses
// V row k0 + s/4, columns d0 + 4 (s%4).., lane j receives V[k0..k0+3][d0+j],
// a column of V: the A operand's four keys. Two such reads give a lane its
// 8 keys, placed in the accumulator order of P^T ({4h..4h+3, 8+4h..8+4h+3}
// for lane half h; MFMA pairs A slot i with B slot i, so only the two sides'
// key orders have to agree).
// Online softmax in base 2 (exponent fma(score, scale*log2(e), -m)), fp32
// state, with the running max m moved lazily (see the loop).
// Workgroups run heaviest (longest causal rows) first across all heads.
#include <algorithm>
#include <vector>

#include "kr_dma.h"
#include "kr_misc.h"

namespace kr {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short AttnS4 __attribute__((ext_vector_type(4)));
typedef uint32_t AttnU2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) AttnS4 *LdsS4;

constexpr int kKvBlk = 64;

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
    // workgroup -> (item, head): xcds 0 = b / HQ, b % HQ; otherwise the 8
    // XCDs (workgroup b runs on XCD b % 8) are shared out by kv head so that
    // one XCD's L2 holds the keys and values of only its own kv heads
    int xcds, nitems;
    AttnItem items[kMaxItems];
};

// Workgroup b -> (item index, query head). XCD x = b % 8 serves kv head
// x / (8 / HKV) when HKV divides 8 (its share of that head's (item, query
// head) units, heaviest items first), or kv heads x, x + 8, ... when 8
// divides HKV. Returns false for the padding workgroups of the last round.
__device__ __forceinline__ bool AttnUnit(const AttnParams &p, int b, int &item, int &h)
{
    if (p.xcds == 0) {
        h = b % p.HQ;
        item = b / p.HQ;
        return true;
    }
    const int x = b % p.xcds, i = b / p.xcds;
    const int gq = p.HQ / p.HKV;  // query heads per kv head
    int kv, u;
    if (p.HKV <= p.xcds) {
        const int r = p.xcds / p.HKV;  // XCDs per kv head
        kv = x / r;
        u = i * r + x % r;
        item = u / gq;
        h = kv * gq + u % gq;
    } else {
        const int per = p.HKV / p.xcds;  // kv heads per XCD
        item = i / (per * gq);
        const int rem = i % (per * gq);
        h = (x + p.xcds * (rem / gq)) * gq + rem % gq;
    }
    return item < p.nitems;
}

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

// LDS slot of 16-byte chunk c in row r of a K / V block (an XOR, so it also
// maps a slot back to its chunk). K (D/8 chunks a row, read 16 rows x one
// chunk per 16 lanes): rows 0..15 of a pass land in 16 distinct slots of the
// 256-byte bank line. V (read by ds_read_b64_tr_b16: 4 rows x 4 chunks per
// 16 lanes): the four rows of a read land in four distinct chunk groups.
template <int D>
__device__ __forceinline__ int KSlot(int r, int c)
{
    if constexpr (D == 128) return c ^ (r & 15);
    else return c ^ ((r >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int VSlot(int r, int c)
{
    if constexpr (D == 128) return c ^ (4 * (r & 3));
    else return c ^ (4 * ((r >> 1) & 1));
}

template <int DT, int D, int KH>
__global__ void __attribute__((amdgpu_flat_work_group_size(256 * KH, 256 * KH), amdgpu_waves_per_eu(2)))
AttnKernel(AttnParams p)
{
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    static_assert(KH == 1 || KH == 2, "one or two key halves");
    constexpr int DCH = D / 8;             // 16-byte chunks per K/V row
    constexpr int DBLK = D / 32;           // 32-wide d blocks of O^T
    constexpr int BLK = kKvBlk * D;        // elements of one K or V block
    constexpr int RPD = 64 / DCH;          // rows per 1 KB DMA block
    constexpr int DPW = kKvBlk / RPD / 4;  // DMA blocks per wave per operand and block
    // two-slot rings [slot][half]: K and V of stage s in slot s & 1
    __shared__ __attribute__((aligned(1024))) uint16_t kring[2][KH][BLK];
    __shared__ __attribute__((aligned(1024))) uint16_t vring[2][KH][BLK];
    __shared__ int last_piece;

    const int hv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 8);  // key half
    const int tid = int(threadIdx.x) & 255;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hf = lane >> 5;
    int item_ix, h;
    if (!AttnUnit(p, int(blockIdx.x), item_ix, h)) return;  // whole workgroup, before any barrier
    const AttnItem item = p.items[item_ix];
    const int qb = item.qb;
    const int q0 = qb * kQBlk;
    const int kvh = h / (p.HQ / p.HKV);
    const int qrow = q0 + wave * 32 + (lane & 31);
    const int wave_q_hi = min(q0 + wave * 32 + 31, p.S - 1);

    uint4 qf[D / 16];
#pragma unroll
    for (int dc = 0; dc < D / 16; ++dc) {
        if (qrow < p.S) {
            qf[dc] = *reinterpret_cast<const uint4 *>(p.q + int64_t(qrow) * p.ldq + int64_t(h) * D + dc * 16 + hf * 8);
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

    // DMA geometry: this wave fills 1 KB blocks wave*DPW .. +DPW-1 of each
    // K and V block; lane -> (row, slot), fetching the chunk the slot holds
    const int drow = wave * DPW * RPD + lane / DCH;
    const int dslot = lane % DCH;
    int koff[DPW], voff[DPW];
#pragma unroll
    for (int j = 0; j < DPW; ++j) {
        const int r = drow + j * RPD;
        koff[j] = r * int(p.ldk) + kvh * D + KSlot<D>(r, dslot) * 8;
        voff[j] = r * int(p.ldv) + kvh * D + VSlot<D>(r, dslot) * 8;
    }
    // block kb of K (or V) -> ring slot buf of this half
    auto dma = [&](const uint16_t *src, int64_t ld, const int (&off)[DPW], uint32_t ring_base, int kb, int buf,
                   bool vswz) {
        const int kv0 = kb * kKvBlk;
        const uint32_t dst = ring_base + uint32_t((buf * KH + hv) * BLK * 2) + uint32_t(wave * DPW) * 1024u;
        if (kv0 + kKvBlk <= p.S) {
            const uint16_t *b0 = src + int64_t(kv0) * ld;
#pragma unroll
            for (int j = 0; j < DPW; ++j) DmaLoad16(b0 + off[j], dst + uint32_t(j) * 1024u);
            return;
        }
        // rows past S re-read row S-1: their keys are masked to -inf, so
        // their P is exactly 0 and their finite K and V contribute nothing
#pragma unroll
        for (int j = 0; j < DPW; ++j) {
            const int r = drow + j * RPD;
            const int kv = min(kv0 + r, p.S - 1);
            const int c = vswz ? VSlot<D>(r, dslot) : KSlot<D>(r, dslot);
            DmaLoad16(src + int64_t(kv) * ld + int64_t(kvh) * D + c * 8, dst + uint32_t(j) * 1024u);
        }
    };
    const uint32_t kring0 = LdsAddr(&kring[0][0][0]);
    const uint32_t vring0 = LdsAddr(&vring[0][0][0]);

    // fragment addresses (elements inside a K / V block)
    // K: lane reads row kh*32 + lane%32, chunk 2 dc + hf
    int kaddr[D / 16];
#pragma unroll
    for (int dc = 0; dc < D / 16; ++dc) {
        const int r = lane & 31;  // (kh*32 keeps r & 15 and (r >> 1) & 7)
        kaddr[dc] = r * D + KSlot<D>(r, 2 * dc + hf) * 8;
    }
    // V^T: lane s of 16-lane group g reads row c*16 + 8 rd + 4 hf + s/4,
    // columns b*32 + 16 (g & 1) + 4 (s & 3)..; the row's low bits (and so
    // the slot's XOR) do not depend on c or rd
    int vaddr[DBLK];
    {
        const int s16 = lane & 15;
        const int g1 = (lane >> 4) & 1;
        const int row = 4 * hf + (s16 >> 2);
#pragma unroll
        for (int b = 0; b < DBLK; ++b) {
            const int col = b * 32 + 16 * g1 + 4 * (s16 & 3);
            vaddr[b] = row * D + VSlot<D>(row, col / 8) * 8 + (col & 7);
        }
    }

    // S^T of one block: 2 halves of 32 keys. The K fragments of d step dc
    // are read KAH steps ahead of their MFMA pair (a rolling window of KAH
    // pairs in flight): left to itself the scheduler reuses one pair of
    // registers and waits out the LDS latency before every pair.
    auto qk = [&](const uint16_t *K, f32x16 (&sacc)[2]) {
        constexpr int NP = D / 16;
        constexpr int KAH = NP < 3 ? NP : 3;
        uint4 kf[2][NP];
        auto rd = [&](int dc) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) kf[kh][dc] = *reinterpret_cast<const uint4 *>(K + kh * 32 * D + kaddr[dc]);
        };
#pragma unroll
        for (int dc = 0; dc < KAH; ++dc) rd(dc);
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[kh][v] = 0.0f;
#pragma unroll
        for (int dc = 0; dc < NP; ++dc) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) sacc[kh] = Mfma<DT>(kf[kh][dc], qf[dc], sacc[kh]);
            if (dc + KAH < NP) rd(dc + KAH);
        }
        // issue order: KAH read pairs, then (MFMA pair, read pair), then the
        // last KAH MFMA pairs (0x100 DS read, 0x008 MFMA)
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * KAH, 0);
#pragma unroll
        for (int i = 0; i < NP - KAH; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * KAH, 0);
    };
    // causal / past-S mask of one block's raw scores: register v of half kh
    // holds key kv0 + kh*32 + 8 (v/4) + 4 hf + v%4, masked to -inf when that
    // exceeds min(qrow, S-1): one compare with a constant
    auto mask = [&](f32x16 (&sacc)[2], int kv0) {
        if (kv0 + kKvBlk - 1 > q0 + wave * 32 || kv0 + kKvBlk > p.S) {
            const int lim = min(qrow, p.S - 1) - kv0 - 4 * hf;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    sacc[kh][v] = kh * 32 + 8 * (v >> 2) + (v & 3) > lim ? -INFINITY : sacc[kh][v];
        }
    };
    // softmax of one block's masked scores -> P^T packed to 16 bits (pf[c]:
    // keys of 16-key step c in the accumulator order), running (m, l);
    // returns the O rescale factor (1 unless the row max moved). The row max
    // is taken on raw scores, before scaling (scale > 0).
    auto softmax = [&](f32x16 (&sacc)[2], uint4 (&pf)[4]) -> float {
        // row max as a tree. Head size 128: 3-input steps in IEEE maximum
        // (v_maximum3_f32 needs no quieting of its inputs, while fmaxf's
        // maxnum first canonicalizes every MFMA result in IEEE mode: 18
        // instructions per block instead of 46). Head size 64 keeps fmaxf,
        // which measured faster there. Both equal on the finite and -inf
        // scores here.
        auto mx2 = [](float a, float b) {
            if constexpr (D == 64) {
                return fmaxf(a, b);
            } else {
                return __builtin_elementwise_maximum(a, b);
            }
        };
        float mx[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int kh = t >> 1, v0 = (t & 1) * 8;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = sacc[kh][v0 + e];
            if constexpr (D == 64) {
                mx[t] = mx2(mx2(mx2(x[0], x[1]), mx2(x[2], x[3])), mx2(mx2(x[4], x[5]), mx2(x[6], x[7])));
            } else {
                mx[t] = mx2(mx2(mx2(mx2(x[0], x[1]), x[2]), mx2(mx2(x[3], x[4]), x[5])), mx2(x[6], x[7]));
            }
        }
        float mloc = mx2(mx2(mx[0], mx[1]), mx2(mx[2], mx[3]));
        // lanes l and l ^ 32 hold the same query: v_permlane32_swap hands
        // every lane both halves' values (no LDS round trip)
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
            mloc = mx2(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * p.scale_log2;
        }
        // lazy rescale: the row's reference max m moves only when a score
        // exceeds it by more than 2^8 (so p = 2^(s - m) <= 256, exact in
        // range for bf16 P and fp32 sums); the wave skips the O rescale
        // when no row moved. O / l is unchanged: both carry the same m.
        const bool move = mloc > m + 8.0f;
        const float mnew = move ? mloc : m;
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = move ? __builtin_amdgcn_exp2f(m - msub) : 1.0f;
        float ls[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int kh = c >> 1, vb = (c & 1) * 8;
            float pv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kh][vb + e], p.scale_log2, -msub));
                ls[e & 3] = c == 0 && e < 4 ? pv[e] : ls[e & 3] + pv[e];
            }
            pf[c] = make_uint4(Pack2<DT>(pv[0], pv[1]), Pack2<DT>(pv[2], pv[3]), Pack2<DT>(pv[4], pv[5]),
                               Pack2<DT>(pv[6], pv[7]));
        }
        l = l * alpha + ((ls[0] + ls[1]) + (ls[2] + ls[3]));
        m = mnew;
        return (__builtin_amdgcn_read_exec() & __ballot(move)) != 0 ? alpha : 1.0f;
    };
    // O^T += V^T . P^T of one block
    auto pv = [&](const uint16_t *V, const uint4 (&pf)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int b = 0; b < DBLK; ++b) {
                const AttnS4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (LdsS4)(const_cast<uint16_t *>(V) + c * 16 * D + vaddr[b]));
                const AttnS4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (LdsS4)(const_cast<uint16_t *>(V) + (c * 16 + 8) * D + vaddr[b]));
                // whole-vector casts: element swizzles of the read's result
                // (lo.zw) have been lowered as copies of its low dword
                const AttnU2 a = __builtin_bit_cast(AttnU2, lo), z = __builtin_bit_cast(AttnU2, hi);
                oacc[b] = Mfma<DT>(make_uint4(a.x, a.y, z.x, z.y), pf[c], oacc[b]);
            }
        }
    };
    auto rescale = [&](float alpha) {
        if (__builtin_expect(__ballot(alpha != 1.0f) != 0, 0)) {
#pragma unroll
            for (int b = 0; b < DBLK; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v) oacc[b][v] *= alpha;
        }
    };

    // Stage s: this half's block kb_lo + s*KH + hv; K and V of stage s+1 are
    // fetched into the other ring slot while stage s is computed.
    const int kb_lo = item.kb_lo, kb_hi = item.kb_hi;
    const int ns = (kb_hi - kb_lo + KH - 1) / KH;
    dma(p.k, p.ldk, koff, kring0, kb_lo + hv, 0, false);
    dma(p.v, p.ldv, voff, vring0, kb_lo + hv, 0, true);
    KR_WAIT_VM(0);
    __syncthreads();
    for (int st = 0; st < ns; ++st) {
        const int kb = kb_lo + st * KH + hv;
        if (st + 1 < ns) {  // the other slot was last read before the previous barrier
            dma(p.k, p.ldk, koff, kring0, kb + KH, (st + 1) & 1, false);
            dma(p.v, p.ldv, voff, vring0, kb + KH, (st + 1) & 1, true);
        }
        // else: the block is past this item's range (odd block count) or
        // entirely in this wave's future
        if (kb < kb_hi && kb * kKvBlk <= wave_q_hi) {
            f32x16 sacc[2];
            qk(kring[st & 1][hv], sacc);
            mask(sacc, kb * kKvBlk);
            uint4 pf[4];
            // Two independent 4-wave workgroups share each CU (KH 1): the
            // wave in its softmax takes issue priority over the other
            // workgroup's wave on its SIMD (measured at head size 128,
            // 4096 x 32 heads: 169-176 against 181-187 us p50, 8192 x 32
            // 612-617 against 616-630; neutral at head size 64 and for the
            // 8-wave kernel, whose barrier keeps its waves in phase).
            if constexpr (KH == 1 && D == 128) __builtin_amdgcn_s_setprio(2);
            rescale(softmax(sacc, pf));
            if constexpr (KH == 1 && D == 128) __builtin_amdgcn_s_setprio(0);
            pv(vring[st & 1][hv], pf);
        }
        KR_WAIT_VM(0);  // this wave's DMA of the next stage has landed
        __syncthreads();
    }

    if constexpr (KH == 2) {
        // waves 4..7 hand their (O, m, l) to waves 0..3 of the same queries
        // through the rings (free: the loop ended on a barrier), lane-major
        // so that a wave's 64 lanes touch 64 consecutive words
        constexpr int NE = DBLK * 16;
        static_assert(4 * NE * 64 * 4 <= int(sizeof(kring)) && 4 * 2 * 64 * 4 <= int(sizeof(vring)), "merge area");
        float *mg = reinterpret_cast<float *>(&kring[0][0][0]) + wave * NE * 64 + lane;
        float *ml = reinterpret_cast<float *>(&vring[0][0][0]) + wave * 2 * 64 + lane;
        if (hv == 1) {
#pragma unroll
            for (int b = 0; b < DBLK; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v) mg[(b * 16 + v) * 64] = oacc[b][v];
            ml[0] = m;
            ml[64] = l;
        }
        __syncthreads();
        if (hv == 0) {
            const float m1 = ml[0];
            const float mn = fmaxf(m, m1);
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float a0 = __builtin_amdgcn_exp2f(m - ms), a1 = __builtin_amdgcn_exp2f(m1 - ms);
            l = __builtin_fmaf(ml[64], a1, l * a0);
#pragma unroll
            for (int b = 0; b < DBLK; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v) oacc[b][v] = __builtin_fmaf(mg[(b * 16 + v) * 64], a1, oacc[b][v] * a0);
            m = mn;
        }
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
        if (hv == 0) {
#pragma unroll
            for (int b = 0; b < DBLK; ++b)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    __hip_atomic_store(part(item.piece, b * 4 + v / 4, v % 4), oacc[b][v], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(part(item.piece, NCH - 1, 0), m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(part(item.piece, NCH - 1, 1), l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial is written
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int32_t *c = p.cnt + int64_t(item.sid) * p.HQ + h;
            const int32_t t = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_piece = t == item.pieces - 1;
            if (last_piece) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last_piece) return;  // the whole workgroup leaves together
        // the partials were stored at agent scope (device-coherent) before
        // the other pieces' tickets; acquire at agent scope so no stale line
        // of this CU's caches serves the reads below
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (hv != 0) return;  // no barrier follows
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
    if (hv != 0) return;
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

namespace {

// KR_ATTN_KH: 1 or 2 forces the key halves per workgroup; 0 (default) picks
int AttnKhEnv()
{
    static const int v = [] {
        const char *e = std::getenv("KR_ATTN_KH");
        const int k = e != nullptr ? std::atoi(e) : 0;
        return k == 1 || k == 2 ? k : 0;
    }();
    return v;
}

template <int DT, int D, int KH>
const void *AttnFn()
{
    return reinterpret_cast<const void *>(&AttnKernel<DT, D, KH>);
}

const void *AttnKernelFor(int dtype, int D, int kh)
{
    const bool bf = dtype == kBF16;
    if (D == 128) {
        if (kh == 2) return bf ? AttnFn<kBF16, 128, 2>() : AttnFn<kF16, 128, 2>();
        return bf ? AttnFn<kBF16, 128, 1>() : AttnFn<kF16, 128, 1>();
    }
    if (kh == 2) return bf ? AttnFn<kBF16, 64, 2>() : AttnFn<kF16, 64, 2>();
    return bf ? AttnFn<kBF16, 64, 1>() : AttnFn<kF16, 64, 1>();
}

}  // namespace

int AttnCus()
{
    static const int v = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    return v;
}

// Resident workgroups of the bf16 kernel (head_dim D, kh key halves) on the
// device: CUs times workgroups per CU, as the runtime's occupancy calculator
// gives them (the LDS rings of the 8-wave kernel at D 128 leave room for one
// per CU, the 4-wave kernel's for two).
int AttnSlots(int D, int kh)
{
    static int cache[2][2] = {{0, 0}, {0, 0}};
    int &v = cache[D == 128 ? 1 : 0][kh - 1];
    if (v == 0) {
        int per = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, AttnKernelFor(kBF16, D, kh), 256 * kh, 0) != hipSuccess ||
            per < 1)
            per = kh == 1 ? 2 : 1;
        v = AttnCus() * per;
    }
    return v;
}

// Key halves: 2 (8 waves; the longest causal row walked in half the stages,
// one workgroup per CU) while the 4-wave grid fits the device's resident
// slots in one round, so that its longest rows would set the time; 1 (4
// waves, two independent workgroups per CU) for larger grids, which the
// heaviest-first order balances on its own. Measured on MI355X, causal,
// D 128: 2048 x 28 heads 61 (kh 2) vs 67 us (kh 1); 4096 x 32 heads 193
// vs 177 us.
int AttnKh(int S, int HQ, int D)
{
    if (AttnKhEnv() != 0) return AttnKhEnv();
    const int64_t grid = int64_t((S + kQBlk - 1) / kQBlk) * HQ;
    return grid <= AttnSlots(D, 1) ? 2 : 1;
}

void AttnSplitNeeds(int S, int HQ, int D, size_t *ws_bytes, int *counters)
{
    *ws_bytes = 0;
    *counters = 0;
    if (S <= 0 || HQ <= 0 || (D != 64 && D != 128)) return;
    // Split only a grid of at most half as many workgroups as CUs: a fuller
    // grid is bound by the CUs' throughput, not by its longest row, and the
    // 8-wave kernel already halves that row (measured on MI355X, causal:
    // 2048 x 28 heads D 128 60 us unsplit vs 61 split, 2048 x 14 heads D 64
    // 37 vs 52, 4096 x 32 heads D 128 180 vs 196).
    // KR_ATTN_SPLIT=1 splits whatever the grid (for timing the policy).
    static const bool force = [] {
        const char *e = std::getenv("KR_ATTN_SPLIT");
        return e != nullptr && std::atoi(e) == 1;
    }();
    if (!force && int64_t((S + kQBlk - 1) / kQBlk) * HQ * 2 > AttnCus()) return;
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
    // XCD-aware order where the kv heads share out evenly over 8 XCDs
    // (KR_ATTN_XCD=0 keeps the plain order)
    static const bool xcd_off = [] {
        const char *e = std::getenv("KR_ATTN_XCD");
        return e != nullptr && std::atoi(e) == 0;
    }();
    const int nit = int(pl.items.size());
    p.nitems = nit;
    p.xcds = !xcd_off && (8 % HKV == 0 || HKV % 8 == 0) ? 8 : 0;
    unsigned nwg = unsigned(nit) * unsigned(HQ);
    if (p.xcds != 0) nwg = 8u * unsigned((int64_t(nit) * HQ + 7) / 8);
    const dim3 grid(nwg);
    if (dtype != kBF16 && dtype != kF16) throw std::runtime_error("attention: dtype must be bf16 or f16");
    if (D != 128 && D != 64) throw std::runtime_error("attention: head_dim must be 64 or 128");
    const int kh = AttnKh(S, HQ, D);
    void *args[] = {&p};
    Check(hipLaunchKernel(AttnKernelFor(dtype, D, kh), grid, dim3(256 * kh), args, 0, stream), "attention launch");
    Check(hipGetLastError(), "attention launch");
}

}  // namespace kr
