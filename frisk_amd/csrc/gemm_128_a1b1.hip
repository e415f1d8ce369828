// The 128x128-tile MFMA GEMM (gemm_128.h) for trans_a = 1, trans_b = 1:
// A stored [K, M], B stored [N, K].
#include "gemm_128.h"

namespace frisk {
template hipError_t gemm_128_layout<true, false>(const GemmArgs&, hipStream_t);
template hipError_t gemm_128_grid_layout<true, false>(const GemmArgs&, hipStream_t);
template hipError_t gemm_128_split_layout<true, false>(const GemmArgs&, int, int64_t, void*,
                                                   hipStream_t);
}  // namespace frisk
