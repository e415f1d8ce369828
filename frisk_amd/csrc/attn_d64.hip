// head_dim 64 variants of the flash-attention forward (attn.h).
#include "attn.h"

namespace frisk {
hipError_t attn_fwd_d64(const AttnArgs& a, hipStream_t s) { return attn_fwd_dispatch<64>(a, s); }
}  // namespace frisk
