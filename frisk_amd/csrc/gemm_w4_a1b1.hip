// The 256x256-tile MFMA GEMM (gemm_w4.h) for trans_a = 1, trans_b = 1:
// A stored [K, M], B stored [N, K].
#include "gemm_w4.h"

namespace frisk {
template hipError_t gemm_w4_layout<true, false>(const GemmArgs&, hipStream_t);
template hipError_t gemm_w4_split_layout<true, false>(const GemmArgs&, int, int64_t, void*,
                                                  hipStream_t);
}  // namespace frisk
