// Construction helpers, accessors and contracts of the frisk tile ops.
#pragma once

#include "ir.h"

namespace fir {

// Execution thread counts accepted by frisk.parallel and the execution
// attributes (FriskOps.cpp:41-44).
bool isSupportedExecutionThreadCount(int64_t threads);

// Element type named by the builder's dtype strings ("fp16", "bf16", "fp32",
// "fp64", "e4m3fn", "e5m2", plus the integer tiles "int8", "int32").
// Throws InvalidArgument("invalid float type") for anything else, like the
// reference's alloc/fill builders (ffi/ir.cpp:399-413, 439-455).
Type dtypeToType(Context* ctx, const std::string& dtype);

// GEMM operand contract of LegacyImportSemantics.cpp:11-46, widened for the
// MI355X matrix cores: besides C == A/B dtype and f16/bf16 -> f32, fp8
// (e4m3fn/e5m2) inputs may accumulate into f32/bf16/f16 C and int8 inputs
// into i32 C.  Returns the first violated rule ("legacy-gemm-shape: ..." or
// "legacy-gemm-type: ...").
std::optional<std::string> legacyGemmValidationError(Type a, Type b, Type c, bool transA,
                                                     bool transB, int64_t m, int64_t n, int64_t k);

// ---- builders (insert at the builder's insertion point) --------------------
Operation* createModule(Builder& b);
Operation* lookupSymbol(Operation* module, const std::string& name);
Operation* createKernel(Builder& b, Operation* module, const std::string& name, Type fnType);
Block* addKernelEntryBlock(Operation* kernel);
Operation* createParallel(Builder& b, const std::vector<int64_t>& grid, int64_t threads);
Block* addParallelEntryBlock(Operation* parallel);
Operation* createBlockOp(Builder& b, const std::vector<int64_t>& ranges,
                         const std::function<void(const std::vector<Value>&)>& body);
Operation* createFor(Builder& b, int64_t lower, int64_t upper, int64_t step,
                     const std::function<void(Value)>& body);
Operation* createEnd(Builder& b);
Operation* createGemm(Builder& b, Value A, Value B, Value C, bool transA, bool transB,
                      bool clearAccum, const std::optional<std::string>& legacySemantics);
Operation* createAllocBuffer(Builder& b, const std::vector<int64_t>& shape, Type elem,
                             MemorySpace space, int64_t alignment);
Operation* createCopy(Builder& b, Value src, Value dst, const std::vector<Value>& srcIdx,
                      const std::vector<Value>& dstIdx, AffineMap srcMap, AffineMap dstMap,
                      std::vector<int64_t> srcExtents, std::vector<int64_t> dstExtents);
Operation* createFill(Builder& b, Value memref, Attribute value);
Operation* createReduce(Builder& b, Value src, Value dst, const std::string& kind, int64_t dim,
                        bool clear, const std::optional<std::string>& legacySemantics);
Operation* createConstant(Builder& b, Attribute value, Type type);
Operation* createFunc(Builder& b, const std::string& name, Type fnType);
Block* addFuncEntryBlock(Operation* func);
Operation* createReturn(Builder& b, const std::vector<Value>& vals);

// Copy helpers matching CopyOp::build (FriskOps.cpp:553-596): whole-tile
// copies when the index lists are empty, identity maps otherwise, and
// source extents = destination shape right-aligned (leading 1s).
std::vector<int64_t> defaultCopySrcExtents(Type src, Type dst);

// ---- accessors --------------------------------------------------------------
struct CopyParts {
  Value src, dst;
  std::vector<Value> srcIdx, dstIdx;
  AffineMap srcMap, dstMap;
  std::vector<int64_t> srcExtents, dstExtents;
};
CopyParts copyParts(Operation* copy);
std::vector<int64_t> i64Array(Operation* op, const std::string& name);

// Per-op contract check (no recursion).  Returns the diagnostic message
// without the "'name' op " prefix, or nullopt.
std::optional<std::string> verifyOpContract(Operation* op);

}  // namespace fir
