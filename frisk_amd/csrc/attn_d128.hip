// head_dim 128 variants of the flash-attention forward (attn.h).
#include "attn.h"

namespace frisk {
hipError_t attn_fwd_d128(const AttnArgs& a, hipStream_t s) { return attn_fwd_dispatch<128>(a, s); }
}  // namespace frisk
