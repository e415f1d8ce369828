// The 128x128-tile MFMA GEMM (gemm_128.h) for trans_a = 0, trans_b = 0:
// A stored [M, K], B stored [K, N].
#include "gemm_128.h"

namespace frisk {
template hipError_t gemm_128_layout<false, true>(const GemmArgs&, hipStream_t);
template hipError_t gemm_128_grid_layout<false, true>(const GemmArgs&, hipStream_t);
template hipError_t gemm_128_split_layout<false, true>(const GemmArgs&, int, int64_t, void*,
                                                   hipStream_t);
}  // namespace frisk
