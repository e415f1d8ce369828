// head_dim 32 variants of the flash-attention forward (attn.h).
#include "attn.h"

namespace frisk {
hipError_t attn_fwd_d32(const AttnArgs& a, hipStream_t s) { return attn_fwd_dispatch<32>(a, s); }
}  // namespace frisk
