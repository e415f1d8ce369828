// The 256x256-tile MFMA GEMM (gemm_w4.h) for trans_a = 0, trans_b = 0:
// A stored [M, K], B stored [K, N].
#include "gemm_w4.h"

namespace frisk {
template hipError_t gemm_w4_layout<false, true>(const GemmArgs&, hipStream_t);
template hipError_t gemm_w4_split_layout<false, true>(const GemmArgs&, int, int64_t, void*,
                                                  hipStream_t);
}  // namespace frisk
