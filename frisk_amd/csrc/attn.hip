// Flash-attention forward (placeholder until the MFMA kernel lands).
#include "kernels.h"

namespace frisk {
hipError_t attn_fwd_d128(const AttnArgs&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace frisk
