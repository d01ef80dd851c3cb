// mixed_body.h - device body of the one-launch mixed step: workgroups
// [0, pf_groups) run the dense prefill's work list, the rest the stream-K
// decode of the single-token rows.  Included by mixed.hip and by the
// code-object entries (module_entry.hip).
#pragma once
#include "attention_body.h"
#include "prefill_body.h"

namespace pam {

static_assert(kPrefillWaves % kMfmaWaves == 0, "the decode part runs whole stream-K units");
static_assert(kMixedMaxRows <= kStreamKMaxRows, "decode rows of a mixed launch");

template <typename KV>
__device__ __forceinline__ void mixed_body(const AttnParams &p) {
    const int b = blockIdx.x;  // workgroup-uniform branch: every barrier below is reached by all waves
    if (b < p.pf_groups)
        prefill_body<128, kPrefillRB, false, KV>(p);
    else
        streamk_body<KV, 128, kBlkTile, false, kPrefillWaves, kMixedMaxRows>(p, b - p.pf_groups,
                                                                             (int)gridDim.x - p.pf_groups);
}

}  // namespace pam
