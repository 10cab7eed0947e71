// Causal GQA flash attention on CDNA4 MFMA (BSND layout).
//
// Replaces the reference's aclnnFlashAttentionScore call (FlashN,
// exec/qwen_main.cpp:591-614: scale 1/sqrt(D), keepProb 1, sparseMode 3 with
// the upper-triangular mask of MakeMask :487-497).
//
// One workgroup = 128 queries of one head (4 waves x 32 queries); keys and
// values stream through LDS in blocks of 64. The kernel computes the
// transposed products so that every operand lands where the next MFMA wants
// it, with no cross-lane shuffles of P:
//   S^T = K . Q^T   (32x32x16: A = K rows from LDS, B = Q rows in registers)
//       -> lane l holds query l%32 and 16 keys of each 32-key half; the row
//          max / sum over keys is a lane-local loop plus one xor-32 shuffle.
//   O^T += V^T . P^T (A = V^T from a transposed LDS copy, B = P^T straight
//          from the S^T accumulators after rounding to 16 bits).
// MFMA pairs A slot s with B slot s, so the key order inside a 16-key step
// only has to agree between V^T and P^T; it is the accumulator's own row
// order {4h..4h+3, 8+4h..8+4h+3}.
// Online softmax in base 2 (scores pre-scaled by scale*log2(e)), fp32 state.
#include "kr_misc.h"

namespace kr {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kKvBlk = 64;
constexpr int kQBlk = 128;

struct AttnParams {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    uint16_t *o;
    int64_t ldq, ldk, ldv, ldo;  // row strides (elements) of the [S, heads*D] views
    int S, HQ, HKV;
    float scale_log2;
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

// 8-byte unit u (4 keys) of row d of V^T.
__device__ __forceinline__ int VSwz(int d, int u) { return u ^ (d & 15); }

template <int DT, int D>
__global__ void __launch_bounds__(256) AttnKernel(AttnParams p)
{
    constexpr int DCH = D / 8;
    constexpr int DBLK = D / 32;
    __shared__ __attribute__((aligned(16))) uint16_t Ks[kKvBlk * D];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[D * kKvBlk];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hf = lane >> 5;
    const int h = blockIdx.y;
    const int nqb = (p.S + kQBlk - 1) / kQBlk;
    const int qb = nqb - 1 - int(blockIdx.x);  // longest causal rows first
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

    const int q_hi = min(q0 + kQBlk - 1, p.S - 1);
    const int nkb = q_hi / kKvBlk + 1;

    for (int kb = 0; kb < nkb; ++kb) {
        const int kv0 = kb * kKvBlk;
        __syncthreads();
        for (int t = tid; t < kKvBlk * DCH; t += 256) {
            const int r = t / DCH, c = t % DCH;
            const int kv = kv0 + r;
            uint4 val = make_uint4(0, 0, 0, 0);
            if (kv < p.S) val = *reinterpret_cast<const uint4 *>(p.k + int64_t(kv) * p.ldk + int64_t(kvh) * D + c * 8);
            *reinterpret_cast<uint4 *>(Ks + r * D + KSwz<D>(r, c) * 8) = val;
        }
        for (int t = tid; t < (kKvBlk / 4) * DCH; t += 256) {
            const int g = t / DCH, c = t % DCH;
            U16x8 rows[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kv = kv0 + 4 * g + i;
                if (kv < p.S) {
                    rows[i] = LoadU16x8(p.v + int64_t(kv) * p.ldv + int64_t(kvh) * D + c * 8);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) rows[i].v[e] = 0;
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = c * 8 + e;
                uint2 w;
                w.x = uint32_t(rows[0].v[e]) | (uint32_t(rows[1].v[e]) << 16);
                w.y = uint32_t(rows[2].v[e]) | (uint32_t(rows[3].v[e]) << 16);
                *reinterpret_cast<uint2 *>(Vt + d * kKvBlk + VSwz(d, g) * 4) = w;
            }
        }
        __syncthreads();
        if (kv0 > wave_q_hi) continue;  // block entirely in this wave's future

        f32x16 sacc[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[kh][v] = 0.0f;
            const int r = kh * 32 + (lane & 31);
#pragma unroll
            for (int dc = 0; dc < D / 16; ++dc) {
                const uint4 kf = *reinterpret_cast<const uint4 *>(Ks + r * D + KSwz<D>(r, dc * 2 + hf) * 8);
                sacc[kh] = Mfma<DT>(kf, qf[dc], sacc[kh]);
            }
        }

        float mloc = -INFINITY;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int kv = kv0 + kh * 32 + 8 * (v >> 2) + 4 * hf + (v & 3);
                float s = sacc[kh][v] * p.scale_log2;
                if (kv > qrow || kv >= p.S) s = -INFINITY;
                sacc[kh][v] = s;
                mloc = fmaxf(mloc, s);
            }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float mnew = fmaxf(m, mloc);
        const float msub = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = exp2f(m - msub);
        float lsum = 0.0f;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float pv = exp2f(sacc[kh][v] - msub);
                sacc[kh][v] = pv;
                lsum += pv;
            }
        l = l * alpha + lsum;
        m = mnew;
#pragma unroll
        for (int b = 0; b < DBLK; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[b][v] *= alpha;

#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int kh = c >> 1;
            const int vb = (c & 1) * 8;
            uint32_t pw[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                pw[s] = uint32_t(Elem<DT>::Store(sacc[kh][vb + 2 * s])) |
                        (uint32_t(Elem<DT>::Store(sacc[kh][vb + 2 * s + 1])) << 16);
            }
            const uint4 pf = make_uint4(pw[0], pw[1], pw[2], pw[3]);
#pragma unroll
            for (int b = 0; b < DBLK; ++b) {
                const int d = b * 32 + (lane & 31);
                const uint2 lo = *reinterpret_cast<const uint2 *>(Vt + d * kKvBlk + VSwz(d, 4 * c + hf) * 4);
                const uint2 hi = *reinterpret_cast<const uint2 *>(Vt + d * kKvBlk + VSwz(d, 4 * c + 2 + hf) * 4);
                oacc[b] = Mfma<DT>(make_uint4(lo.x, lo.y, hi.x, hi.y), pf, oacc[b]);
            }
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

void AttnLaunch(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                void *out, int64_t ldo, int S, int HQ, int HKV, int D, float scale, hipStream_t stream)
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
    p.S = S;
    p.HQ = HQ;
    p.HKV = HKV;
    p.scale_log2 = scale * 1.4426950408889634f;
    const dim3 grid((S + kQBlk - 1) / kQBlk, HQ);
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
