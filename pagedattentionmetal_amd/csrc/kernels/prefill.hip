// prefill.hip - dense chunked prefill for gfx950 (placeholder dispatch until the
// MFMA tile kernel lands; the row kernels in attention.hip serve every prefill).
#include "kernels.h"

namespace pam {

bool prefill_mfma_supported(int32_t, int32_t, int32_t) { return false; }

hipError_t launch_prefill_mfma(const AttnParams &, hipStream_t) { return hipErrorNotSupported; }

}  // namespace pam
