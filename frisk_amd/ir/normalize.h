// Legacy tile ops -> tensor-form ops (the reference's
// `frisk-normalize-layout-ir` pass, LegacyFragmentNormalization.cpp).
#pragma once

#include <string>

#include "ir.h"

namespace fir {

// Rewrite `module` in place: Local alloc_buffer fragments become SSA tensor
// values (fill -> arith.constant, gemm -> frisk.mma, reduce ->
// frisk.reduce_tensor [+ arith merge], copy -> tile_load / tile_store),
// frisk.for loops that carry fragments become scf.for with iter_args, and
// Shared/Global allocations become memref.alloc.  Returns "" on success or
// the diagnostic of the first violated contract (the module may then be
// partially rewritten, as with a failed MLIR pass).
std::string normalizeLegacyFragments(Operation* module);

// The MFMA target every frisk.mma must be lowered for.
inline const char* kCdna4Target = "gfx950";

}  // namespace fir
