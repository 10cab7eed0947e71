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
// n bf16 values of about N(0, std^2), a function of (seed, index) only.
void RandBf16Launch(void *p, int64_t n, uint32_t seed, float std, hipStream_t stream);

// Causal GQA attention, BSND layout: q [S, HQ, D], k/v [S, HKV, D],
// out [S, HQ, D], each with its own row stride (elements; 0 = packed);
// query head h reads key/value head h / (HQ/HKV); scores scaled by `scale`;
// key j visible to query i iff j <= i.
// With `split` (a workspace of AttnSplitNeeds' size; counters zero before
// the first launch, left zero by every launch, owned by one stream), query
// rows longer than 16 key blocks (KR_ATTN_CAP) are cut into up to 4 pieces
// that run as separate workgroups and are summed in piece order by the last
// to finish: the grid's critical path follows the average row instead of the
// longest. Bits depend on (S, the cap) only.
struct AttnSplit {
    float *ws = nullptr;
    size_t ws_bytes = 0;
    int32_t *cnt = nullptr;
    int cnt_len = 0;
};
void AttnSplitNeeds(int S, int HQ, int D, size_t *ws_bytes, int *counters);
void AttnLaunch(int dtype, const void *q, int64_t ldq, const void *k, int64_t ldk, const void *v, int64_t ldv,
                void *out, int64_t ldo, int S, int HQ, int HKV, int D, float scale, hipStream_t stream,
                const AttnSplit *split = nullptr);

}  // namespace kr
