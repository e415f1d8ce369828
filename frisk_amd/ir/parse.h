// Parser of the textual tile IR: the custom assembly printOp emits (the
// reference's frisk op formats, FriskOps.cpp / FriskOps.td /
// FriskLayoutOps.td, and the builtin / arith / memref / scf / func forms used
// with them) and MLIR's generic operation form `"name"(...) ... : (...) ->
// (...)` for everything else.  It is the input side of the frisk-opt-like
// command-line driver (frisk_amd/opt.py), whose reference counterpart is
// tools/frisk-opt/frisk-opt.cpp (MlirOptMain over the frisk passes).
#pragma once

#include <string>

#include "ir.h"

namespace fir {

// Parse one `module { ... }` (or a bare sequence of top-level operations,
// which is wrapped in a module) into a detached module owned by `ctx`.
// Malformed input throws InvalidArgument("<line>:<col>: <message>").
Operation* parseModule(Context* ctx, const std::string& text);

}  // namespace fir
