// Host interface of the prefill support kernels (kr_misc.hip) and the
// flash-attention kernel (kr_attn.hip).
#pragma once

#include "kr_common.h"

#include <algorithm>

namespace kr {

void EmbedLaunch(const void *table, const int64_t *ids, void *out, int rows, int cols, int64_t vocab,
                 hipStream_t stream);
void RopeLaunch(int dtype, void *x, int64_t ld, int S, int heads, int D, const void *cos_t,
                const void *sin_t, hipStream_t stream);
void TransposeLaunch(const void *src, void *dst, int R, int C, hipStream_t stream);
void FillLaunch(int32_t *p, int64_t n, int32_t v, hipStream_t stream);

// Causal GQA attention, BSND layout: q [S, HQ, D], k/v [S, HKV, D],
// out [S, HQ, D], each with its own row stride (elements; 0 = packed);
// query head h reads key/value head h / (HQ/HKV); scores scaled by `scale`;
// key j visible to query i iff j <= i.
void AttnLaunch(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                void *out, int64_t ldo, int S, int HQ, int HKV, int D, float scale, hipStream_t stream);

}  // namespace kr
