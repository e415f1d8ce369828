// head_dim 16 variants of the flash-attention forward (attn.h).
#include "attn.h"

namespace frisk {
hipError_t attn_fwd_d16(const AttnArgs& a, hipStream_t s) { return attn_fwd_dispatch<16>(a, s); }
}  // namespace frisk
