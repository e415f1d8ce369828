// Builders, accessors and verifiers of the frisk tile ops and of the
// tensor-form layout ops the normalizer emits.
//
// Contracts follow the reference op definitions: FriskOps.td /
// FriskOps.cpp (kernel :76-101, parallel :161-235, block :239-258, for
// :340-360, gemm :406-414, alloc_buffer :456-501, copy :553-680, fill
// :682-696, reduce :720-763), LegacyImportSemantics.cpp:11-46 (gemm
// operands) and FriskLayoutOps.cpp:34-118 (reduce_tensor, mma).
#include "ops.h"

#include <algorithm>
#include <sstream>

namespace fir {

bool isSupportedExecutionThreadCount(int64_t t) {
  return t == 32 || t == 64 || t == 128 || t == 256 || t == 512 || t == 1024;
}

Type dtypeToType(Context* ctx, const std::string& d) {
  if (d == "e4m3fn") return ctx->floatTy(FloatKind::E4M3FN);
  if (d == "e5m2") return ctx->floatTy(FloatKind::E5M2);
  if (d == "fp16") return ctx->floatTy(FloatKind::F16);
  if (d == "bf16") return ctx->floatTy(FloatKind::BF16);
  if (d == "fp32") return ctx->floatTy(FloatKind::F32);
  if (d == "fp64") return ctx->floatTy(FloatKind::F64);
  if (d == "int8") return ctx->integer(8);
  if (d == "int32") return ctx->integer(32);
  throw InvalidArgument("invalid float type");
}

std::optional<std::string> legacyGemmValidationError(Type aT, Type bT, Type cT, bool transA,
                                                     bool transB, int64_t m, int64_t n, int64_t k) {
  if (!aT.isMemRef() || !bT.isMemRef() || !cT.isMemRef())
    return std::string("legacy-gemm-shape: A, B, and C must be memrefs");
  if (aT.rank() != 2 || bT.rank() != 2 || cT.rank() != 2)
    return std::string("legacy-gemm-shape: A, B, and C must have rank 2");
  if (!aT.hasStaticShape() || !bT.hasStaticShape() || !cT.hasStaticShape())
    return std::string("legacy-gemm-shape: A, B, and C must have static shapes");
  if (m <= 0 || n <= 0 || k <= 0)
    return std::string("legacy-gemm-shape: M, N, and K must be positive");
  Type in = aT.elementType(), acc = cT.elementType();
  if (in != bT.elementType())
    return std::string("legacy-gemm-type: A and B must have the same element type");
  const bool same = acc == in;
  const bool halfToF32 = (in.isF16() || in.isBF16()) && acc.isF32();
  const bool fp8 = in.isFloat(FloatKind::E4M3FN) || in.isFloat(FloatKind::E5M2);
  const bool fp8Acc = fp8 && (acc.isF32() || acc.isBF16() || acc.isF16());
  const bool int8Acc = in.isSignlessInteger(8) && acc.isSignlessInteger(32);
  if (!same && !halfToF32 && !fp8Acc && !int8Acc)
    return std::string(
        "legacy-gemm-type: C must match A/B, be f32 for f16/bf16 inputs, f32/bf16/f16 for fp8 "
        "inputs or i32 for i8 inputs");
  const int64_t aM = aT.dim(transA ? 1 : 0), aK = aT.dim(transA ? 0 : 1);
  const int64_t bK = bT.dim(transB ? 1 : 0), bN = bT.dim(transB ? 0 : 1);
  if (aM != m || aK != k || bK != k || bN != n)
    return std::string("legacy-gemm-shape: effective A/B shapes must match M/N/K");
  if (cT.dim(0) != m || cT.dim(1) != n) return std::string("legacy-gemm-shape: C shape must be MxN");
  return std::nullopt;
}

// ============================================================================
// Builders
// ============================================================================
Operation* createModule(Builder& b) {
  Operation* m = b.create("builtin.module", {}, {}, {}, 1);
  m->region(0).emplaceBlock();
  return m;
}

Operation* lookupSymbol(Operation* module, const std::string& name) {
  Block* body = module->body();
  if (!body) return nullptr;
  for (auto& op : body->ops) {
    Attribute s = op->attr("sym_name");
    if (s && s.kind() == AttrKind::String && s->s == name) return op.get();
  }
  return nullptr;
}

Operation* createKernel(Builder& b, Operation* module, const std::string& name, Type fnType) {
  if (Operation* existing = lookupSymbol(module, name)) {
    if (!existing->is("frisk.kernel"))
      throw InvalidArgument("symbol '" + name + "' is not a kernel");
    return existing;
  }
  if (!fnType.isFunction()) throw InvalidArgument("invalid kernel function type");
  return b.create("frisk.kernel", {}, {},
                  {{"function_type", Attribute::typeAttr(fnType)},
                   {"sym_name", Attribute::string(name)}},
                  1);
}

namespace {
Block* newEntryBlock(Operation* op, const std::vector<Type>& argTypes, bool withEnd) {
  Region& r = op->region(0);
  if (!r.empty()) throw InvalidArgument("entry block already exists");
  Block* entry = r.emplaceBlock();
  for (auto& t : argTypes) entry->addArgument(t);
  if (withEnd) entry->pushBack(makeOp(op->ctx, "frisk.end", op->loc, {}, {}));
  return entry;
}
}  // namespace

Block* addKernelEntryBlock(Operation* kernel) {
  Type fn = kernel->attr("function_type")->type;
  return newEntryBlock(kernel, fn.inputs(), true);
}

Operation* createParallel(Builder& b, const std::vector<int64_t>& grid, int64_t threads) {
  // A parallel op is the only op (besides the terminator) of its block
  // (ffi/ir.cpp:363-370).
  Block* blk = b.insertionBlock();
  if (!blk || blk->ops.size() != 1) throw InvalidArgument("invalid parallel create");
  return b.create("frisk.parallel", {}, {},
                  {{"ranges", Attribute::denseI64(grid)},
                   {"threads", Attribute::integer(b.context()->integer(64), threads)}},
                  1);
}

Block* addParallelEntryBlock(Operation* parallel) {
  const size_t dims = i64Array(parallel, "ranges").size();
  return newEntryBlock(parallel, std::vector<Type>(dims, parallel->ctx->index()), true);
}

namespace {
// Build a single-block region op whose body is filled by `fill` with the
// builder pointed at the new block; the op is inserted at the caller's
// insertion point afterwards (the OpBuilder::InsertionGuard pattern of
// FriskOps.cpp:239-258 and :340-360).
Operation* buildWithBody(Builder& b, std::unique_ptr<Operation> op, unsigned numIvs,
                         const std::function<void(const std::vector<Value>&)>& fill) {
  Block* body = op->region(0).emplaceBlock();
  std::vector<Value> ivs;
  for (unsigned i = 0; i < numIvs; ++i) ivs.push_back(body->addArgument(b.context()->index()));
  InsertPoint saved = b.saveInsertionPoint();
  b.setInsertionPointToStart(body);
  try {
    if (fill) fill(ivs);
  } catch (...) {
    b.restoreInsertionPoint(saved);
    throw;
  }
  b.setInsertionPointToEnd(body);
  createEnd(b);
  b.restoreInsertionPoint(saved);
  return b.insert(std::move(op));
}
}  // namespace

Operation* createBlockOp(Builder& b, const std::vector<int64_t>& ranges,
                         const std::function<void(const std::vector<Value>&)>& body) {
  auto op = makeOp(b.context(), "frisk.block", b.loc(), {}, {},
                   {{"ranges", Attribute::denseI64(ranges)}}, 1);
  return buildWithBody(b, std::move(op), (unsigned)ranges.size(), body);
}

Operation* createFor(Builder& b, int64_t lower, int64_t upper, int64_t step,
                     const std::function<void(Value)>& body) {
  Type i64 = b.context()->integer(64);
  auto op = makeOp(b.context(), "frisk.for", b.loc(), {}, {},
                   {{"lower", Attribute::integer(i64, lower)},
                    {"step", Attribute::integer(i64, step)},
                    {"upper", Attribute::integer(i64, upper)}},
                   1);
  return buildWithBody(b, std::move(op), 1, [&](const std::vector<Value>& ivs) {
    if (body) body(ivs[0]);
  });
}

Operation* createEnd(Builder& b) { return b.create("frisk.end", {}, {}); }

Operation* createGemm(Builder& b, Value A, Value B, Value C, bool transA, bool transB,
                      bool clearAccum, const std::optional<std::string>& legacySemantics) {
  // Shape derivation and contract of ffi/ir.cpp:323-350.
  Type aT = A.type(), bT = B.type();
  if (!aT.isMemRef() || !bT.isMemRef() || aT.rank() != 2 || bT.rank() != 2 ||
      !aT.hasStaticShape() || !bT.hasStaticShape())
    throw InvalidArgument("legacy-gemm-shape: A and B must be static rank-2 memrefs");
  const int64_t m = aT.dim(transA ? 1 : 0), k = aT.dim(transA ? 0 : 1), n = bT.dim(transB ? 0 : 1);
  if (auto err = legacyGemmValidationError(aT, bT, C.type(), transA, transB, m, n, k))
    throw InvalidArgument(*err);
  Type i64 = b.context()->integer(64);
  Operation* op = b.create("frisk.gemm", {A, B, C}, {},
                           {{"K", Attribute::integer(i64, k)},
                            {"M", Attribute::integer(i64, m)},
                            {"N", Attribute::integer(i64, n)},
                            {"clear_accum", Attribute::boolean(clearAccum)},
                            {"policy", Attribute::gemmPolicy(GemmWarpPolicy::Square)},
                            {"transA", Attribute::boolean(transA)},
                            {"transB", Attribute::boolean(transB)}});
  if (legacySemantics) op->setAttr("frisk.legacy_semantics", Attribute::string(*legacySemantics));
  return op;
}

Operation* createAllocBuffer(Builder& b, const std::vector<int64_t>& shape, Type elem,
                             MemorySpace space, int64_t alignment) {
  if (alignment < 0) throw InvalidArgument("alignment must be non-negative");
  for (int64_t d : shape)
    if (d < 0) throw InvalidArgument("alloc_buffer extents must be static and non-negative");
  Type mt = b.context()->memref(shape, elem, AffineMap(), (int64_t)space);
  return b.create("frisk.alloc_buffer", {}, {mt},
                  {{"alignment", Attribute::integer(b.context()->integer(64), alignment)},
                   {"elementType", Attribute::typeAttr(elem)},
                   {"memorySpace", Attribute::memorySpace(space)},
                   {"shape", Attribute::denseI64(shape)}});
}

std::vector<int64_t> defaultCopySrcExtents(Type src, Type dst) {
  const int64_t sr = src.rank(), dr = dst.rank();
  if (sr < dr) throw InvalidArgument("copy source rank must be >= destination rank");
  std::vector<int64_t> ext;
  for (int64_t i = 0; i < sr; ++i) ext.push_back(i < sr - dr ? 1 : dst.dim(i - (sr - dr)));
  return ext;
}

Operation* createCopy(Builder& b, Value src, Value dst, const std::vector<Value>& srcIdx,
                      const std::vector<Value>& dstIdx, AffineMap srcMap, AffineMap dstMap,
                      std::vector<int64_t> srcExtents, std::vector<int64_t> dstExtents) {
  if (!src.type().isMemRef() || !dst.type().isMemRef())
    throw InvalidArgument("copy source and destination must be memrefs");
  Context* ctx = b.context();
  // The three accepted argument combinations of ffi/ir.cpp:418-434; any
  // other mix is rejected (the reference aborts the process there).
  const bool noMaps = !srcMap && !dstMap, bothMaps = srcMap && dstMap;
  const bool noExt = srcExtents.empty() && dstExtents.empty();
  const bool bothExt = !srcExtents.empty() && !dstExtents.empty();
  if (noMaps && noExt) {
    srcMap = srcIdx.empty() ? AffineMap::get(ctx)
                            : AffineMap::multiDimIdentity((unsigned)src.type().rank(), ctx);
    dstMap = dstIdx.empty() ? AffineMap::get(ctx)
                            : AffineMap::multiDimIdentity((unsigned)dst.type().rank(), ctx);
  } else if (!(bothMaps && (noExt || bothExt))) {
    throw InvalidArgument(
        "copy op map error: pass no maps and no extents, both maps, or both maps and both "
        "extents");
  }
  if (srcMap.numInputs() != srcIdx.size())
    throw InvalidArgument("copy op map error: source map inputs must match source indices count");
  if (dstMap.numInputs() != dstIdx.size())
    throw InvalidArgument(
        "copy op map error: destination map inputs must match destination indices count");
  if (noExt) {
    srcExtents = defaultCopySrcExtents(src.type(), dst.type());
    dstExtents = dst.type().shape();
  }
  for (auto& v : srcIdx)
    if (!v.type().isIndex()) throw InvalidArgument("copy indices must have index type");
  for (auto& v : dstIdx)
    if (!v.type().isIndex()) throw InvalidArgument("copy indices must have index type");
  std::vector<Value> operands{src, dst};
  operands.insert(operands.end(), srcIdx.begin(), srcIdx.end());
  operands.insert(operands.end(), dstIdx.begin(), dstIdx.end());
  return b.create("frisk.copy", operands, {},
                  {{"dstExtents", Attribute::denseI64(dstExtents)},
                   {"dstMap", Attribute::affineMap(dstMap)},
                   {"operandSegmentSizes",
                    Attribute::denseI64({1, 1, (int64_t)srcIdx.size(), (int64_t)dstIdx.size()})},
                   {"srcExtents", Attribute::denseI64(srcExtents)},
                   {"srcMap", Attribute::affineMap(srcMap)}});
}

Operation* createFill(Builder& b, Value memref, Attribute value) {
  return b.create("frisk.fill", {memref}, {}, {{"value", value}});
}

Operation* createReduce(Builder& b, Value src, Value dst, const std::string& kind, int64_t dim,
                        bool clear, const std::optional<std::string>& legacySemantics) {
  Operation* op = b.create("frisk.reduce", {src, dst}, {},
                           {{"clear", Attribute::boolean(clear)},
                            {"dim", Attribute::integer(b.context()->integer(64), dim)},
                            {"kind", Attribute::string(kind)}});
  if (legacySemantics) op->setAttr("frisk.legacy_semantics", Attribute::string(*legacySemantics));
  return op;
}

Operation* createConstant(Builder& b, Attribute value, Type type) {
  return b.create("arith.constant", {}, {type}, {{"value", value}});
}

Operation* createFunc(Builder& b, const std::string& name, Type fnType) {
  if (!fnType.isFunction()) throw InvalidArgument("invalid function type");
  return b.create("func.func", {}, {},
                  {{"function_type", Attribute::typeAttr(fnType)},
                   {"sym_name", Attribute::string(name)}},
                  1);
}

Block* addFuncEntryBlock(Operation* func) {
  return newEntryBlock(func, func->attr("function_type")->type.inputs(), false);
}

Operation* createReturn(Builder& b, const std::vector<Value>& vals) {
  return b.create("func.return", vals, {});
}

// ============================================================================
// Accessors
// ============================================================================
std::vector<int64_t> i64Array(Operation* op, const std::string& name) {
  Attribute a = op->attr(name);
  if (!a || a.kind() != AttrKind::DenseI64Array)
    throw InvalidArgument("'" + op->name + "' op has no i64 array attribute " + name);
  return a->ints;
}

CopyParts copyParts(Operation* copy) {
  CopyParts p;
  auto seg = i64Array(copy, "operandSegmentSizes");
  p.src = copy->operand(0);
  p.dst = copy->operand(1);
  for (int64_t i = 0; i < seg[2]; ++i) p.srcIdx.push_back(copy->operand(2 + (unsigned)i));
  for (int64_t i = 0; i < seg[3]; ++i) p.dstIdx.push_back(copy->operand(2 + (unsigned)(seg[2] + i)));
  p.srcMap = copy->attr("srcMap")->map;
  p.dstMap = copy->attr("dstMap")->map;
  p.srcExtents = i64Array(copy, "srcExtents");
  p.dstExtents = i64Array(copy, "dstExtents");
  return p;
}

// ============================================================================
// Contracts
// ============================================================================
namespace {
using Diag = std::optional<std::string>;

bool isPow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// Execution-contract attributes every tile op may carry (FriskOps.cpp:46-68).
Diag verifyExecutionAttributes(Operation* op) {
  if (Attribute p = op->attr("frisk.writer_policy")) {
    if (p.kind() != AttrKind::String || (p->s != "all" && p->s != "first_owner"))
      return std::string("frisk.writer_policy must be all or first_owner");
  }
  for (const char* name : {"frisk.execution_threads", "frisk.vector_bytes"}) {
    Attribute a = op->attr(name);
    if (!a) continue;
    if (a.kind() != AttrKind::Integer || !a->type.isSignlessInteger(64))
      return std::string(name) + " must be an i64 attribute";
    const int64_t n = a->i;
    const bool ok = std::string(name) == "frisk.execution_threads"
                        ? isSupportedExecutionThreadCount(n)
                        : (n == 1 || n == 2 || n == 4 || n == 8 || n == 16);
    if (!ok) return "unsupported " + std::string(name) + " value " + std::to_string(n);
  }
  return std::nullopt;
}

Diag verifyKernelLike(Operation* op) {
  Attribute ft = op->attr("function_type");
  if (!ft || ft.kind() != AttrKind::TypeA) return std::string("requires a 'function_type' attribute");
  if (!ft->type.isFunction()) return std::string("requires a function type");
  Block* body = op->body();
  if (!body) return std::nullopt;  // declaration
  auto ins = ft->type.inputs();
  if (body->numArguments() != ins.size())
    return std::string("region argument count does not match function type");
  for (unsigned i = 0; i < ins.size(); ++i)
    if (body->argument(i).type() != ins[i]) return std::string("region argument type mismatch");
  return std::nullopt;
}

Diag verifyParallel(Operation* op) {
  const int64_t threads = op->intAttr("threads");
  if (!isSupportedExecutionThreadCount(threads))
    return std::string("threads must be one of 32,64,128,256,512,1024");
  auto ranges = i64Array(op, "ranges");
  if (ranges.empty() || std::any_of(ranges.begin(), ranges.end(), [](int64_t n) { return n <= 0; }))
    return std::string("ranges must contain positive static extents");
  Block* body = op->body();
  if (!body || body->numArguments() != ranges.size())
    return std::string("range count must match the region induction arguments");
  for (auto& a : body->args)
    if (!a->type.isIndex()) return std::string("induction arguments must have index type");
  Operation* parent = op->parentOp();
  if (!parent || !parent->is("frisk.kernel")) return std::string("expects parent op 'frisk.kernel'");
  return std::nullopt;
}

Diag verifyGemm(Operation* op) {
  if (op->intAttr("policy") == (int64_t)GemmWarpPolicy::Auto)
    return std::string(
        "Auto policy requires frisk.mma; legacy gemm has deterministic partitioning");
  return legacyGemmValidationError(op->operand(0).type(), op->operand(1).type(),
                                   op->operand(2).type(), op->boolAttr("transA"),
                                   op->boolAttr("transB"), op->intAttr("M"), op->intAttr("N"),
                                   op->intAttr("K"));
}

Diag verifyAlloc(Operation* op) {
  if (op->numResults() != 1 || !op->result(0).type().isMemRef())
    return std::string("result must be a memref type");
  Type mt = op->result(0).type();
  if (mt.shape() != i64Array(op, "shape"))
    return std::string("shape attribute must match result memref shape");
  Attribute et = op->attr("elementType");
  if (!et || et.kind() != AttrKind::TypeA || et->type != mt.elementType())
    return std::string("elementType attribute must match result memref element type");
  Attribute ms = op->attr("memorySpace");
  auto space = mt.memorySpace();
  if (!ms || ms.kind() != AttrKind::MemorySpaceA || !space || (int64_t)*space != ms->i)
    return std::string("memorySpace attribute must match result memref memory space");
  const int64_t align = op->intAttr("alignment");
  if (align < 0) return std::string("alignment must be non-negative");
  if (align > 0 && !isPow2(align)) return std::string("alignment must be a power of 2");
  return std::nullopt;
}

Diag verifyCopy(Operation* op) {
  if (auto d = verifyExecutionAttributes(op)) return d;
  CopyParts p = copyParts(op);
  if (!p.src.type().isMemRef() || !p.dst.type().isMemRef())
    return std::string("source and destination must be memrefs");
  if (p.srcIdx.size() != p.srcMap.numInputs())
    return "expected " + std::to_string(p.srcMap.numInputs()) + " source indices, but got " +
           std::to_string(p.srcIdx.size());
  if (p.dstIdx.size() != p.dstMap.numInputs())
    return "expected " + std::to_string(p.dstMap.numInputs()) + " destination indices, but got " +
           std::to_string(p.dstIdx.size());
  return std::nullopt;
}

Diag verifyFill(Operation* op) {
  if (auto d = verifyExecutionAttributes(op)) return d;
  Type mt = op->operand(0).type();
  if (!mt.isMemRef()) return std::string("fill destination must be a memref");
  Attribute v = op->attr("value");
  if (!v || v.kind() != AttrKind::Float) return std::string("fill value must be a float attribute");
  if (v->type != mt.elementType())
    return "value type " + v->type.str() + " does not match memref element type " +
           mt.elementType().str();
  return std::nullopt;
}

Diag verifyReduce(Operation* op) {
  Type s = op->operand(0).type(), d = op->operand(1).type();
  if (!s.isMemRef() || !d.isMemRef()) return std::string("source and destination must be memref types");
  const int64_t dim = op->intAttr("dim");
  const std::string kind = op->strAttr("kind");
  if (dim < 0 || dim >= s.rank())
    return "dimension " + std::to_string(dim) + " is out of range for source of rank " +
           std::to_string(s.rank());
  if (kind != "add" && kind != "mul" && kind != "min" && kind != "max")
    return "unsupported reduce kind: " + kind + ". Supported: add, mul, min, max";
  if (s.rank() != d.rank() + 1)
    return "destination rank must be one less than source rank. Got: " + std::to_string(d.rank()) +
           " vs " + std::to_string(s.rank());
  for (int64_t i = 0, j = 0; i < s.rank(); ++i) {
    if (i == dim) continue;
    if (s.dim(i) != d.dim(j))
      return "non-reduced dimension mismatch: source[" + std::to_string(i) + "] = " +
             std::to_string(s.dim(i)) + " vs destination[" + std::to_string(j) + "] = " +
             std::to_string(d.dim(j));
    ++j;
  }
  if (s.elementType() != d.elementType())
    return std::string("source and destination must have the same element type");
  return std::nullopt;
}

Diag verifyReduceTensor(Operation* op) {
  Type s = op->operand(0).type(), d = op->result(0).type();
  const std::string kind = op->strAttr("kind");
  const int64_t dim = op->intAttr("dim");
  if (kind != "sum" && kind != "max" && kind != "min")
    return std::string("reduce-shape: kind must be sum/max/min");
  if (!s.isTensor() || !d.isTensor() || s.rank() < 2 || d.rank() != s.rank() - 1 || dim < 0 ||
      dim >= s.rank())
    return std::string("reduce-shape: rank >= 2 and valid axis required");
  Type e = s.elementType();
  if ((!e.isF16() && !e.isBF16() && !e.isF32()) || e != d.elementType())
    return std::string("reduce-shape: requires matching f16/bf16/f32 element types");
  for (Type t : {s, d})
    for (int64_t x : t.shape())
      if (!isPow2(x)) return std::string("reduce-shape: requires static positive power-of-two extents");
  std::vector<int64_t> shape = s.shape();
  shape.erase(shape.begin() + dim);
  if (d.shape() != shape) return std::string("reduce-shape: result must delete the reduction axis");
  if (Attribute t = op->attr("frisk.execution_threads")) {
    if (t.kind() != AttrKind::Integer || !t->type.isSignlessInteger(64) || t->i < 32 ||
        t->i > 1024 || !isPow2(t->i))
      return std::string("reduce-thread-group: requires 32/64/128/256/512/1024 threads");
  }
  return std::nullopt;
}

Diag verifyMma(Operation* op) {
  const int64_t m = op->intAttr("m"), n = op->intAttr("n"), k = op->intAttr("k");
  if (m <= 0 || n <= 0 || k <= 0) return std::string("mma-shape: m/n/k must be positive signless i64");
  Type a = op->operand(0).type(), b = op->operand(1).type(), init = op->operand(2).type(),
       res = op->result(0).type();
  for (Type t : {a, b, init, res}) {
    if (!t.isShaped() || t.rank() != 2 || !t.hasStaticShape() || t.dim(0) <= 0 || t.dim(1) <= 0 ||
        !(t.elementType().isFloat() || t.elementType().isInteger()))
      return std::string("mma-shape: requires positive static rank-2 matrices");
  }
  if (!init.isTensor() || !res.isTensor())
    return std::string("mma-shape: init and result must be tensors");
  if (a.elementType() != b.elementType() || init.elementType() != res.elementType() ||
      init.elementType().bitWidth() < a.elementType().bitWidth())
    return std::string("mma-shape: incompatible input/accumulator element types");
  const bool ta = op->boolAttr("trans_a"), tb = op->boolAttr("trans_b");
  if (a.dim(ta ? 1 : 0) != m || a.dim(ta ? 0 : 1) != k || b.dim(tb ? 1 : 0) != k ||
      b.dim(tb ? 0 : 1) != n || init.shape() != std::vector<int64_t>{m, n} ||
      res.shape() != init.shape())
    return std::string("mma-shape: matrix extents disagree with m/n/k and transpose");
  if (Attribute t = op->attr("frisk.execution_threads")) {
    if (t.kind() != AttrKind::Integer || !t->type.isSignlessInteger(64) || t->i <= 0)
      return std::string("mma-thread-group: expected positive signless i64 threads");
  }
  return std::nullopt;
}

Diag verifyTileLoad(Operation* op) {
  Type m = op->operand(0).type(), t = op->result(0).type();
  if (!m.isMemRef() || !m.hasStaticShape() || !t.isTensor() || m.shape() != t.shape() ||
      m.elementType() != t.elementType())
    return std::string("tile-load: result must be the static source tile as a tensor");
  return std::nullopt;
}

Diag verifyTileStore(Operation* op) {
  Type t = op->operand(0).type(), m = op->operand(1).type();
  if (!m.isMemRef() || !m.hasStaticShape() || !t.isTensor() || m.shape() != t.shape() ||
      m.elementType() != t.elementType())
    return std::string("tile-store: value must be the static target tile as a tensor");
  return std::nullopt;
}

Diag verifyLayoutView(Operation* op) {
  if (op->operand(0).type() != op->result(0).type())
    return std::string("layout-view: result type must equal the source type");
  return std::nullopt;
}

Diag verifyConstant(Operation* op) {
  Attribute v = op->attr("value");
  if (!v) return std::string("requires a 'value' attribute");
  Type rt = op->result(0).type();
  if ((v.kind() == AttrKind::Float || v.kind() == AttrKind::Integer) && v->type != rt)
    return std::string("value type does not match the result type");
  if ((v.kind() == AttrKind::DenseFloat || v.kind() == AttrKind::DenseInt) && v->type != rt)
    return std::string("dense value type does not match the result type");
  return std::nullopt;
}

Diag verifyScfFor(Operation* op) {
  if (op->numOperands() < 3) return std::string("needs lower bound, upper bound and step");
  const unsigned iters = op->numOperands() - 3;
  Block* body = op->body();
  if (!body || body->numArguments() != iters + 1)
    return std::string("region must take the induction variable and one argument per iter_arg");
  if (op->numResults() != iters) return std::string("needs one result per iter_arg");
  for (unsigned i = 0; i < iters; ++i)
    if (op->operand(3 + i).type() != op->result(i).type() ||
        body->argument(1 + i).type() != op->result(i).type())
      return std::string("iter_arg, region argument and result types must agree");
  Operation* y = body->terminator();
  if (!y || !y->is("scf.yield") || y->numOperands() != iters)
    return std::string("body must end in scf.yield of every iter_arg");
  for (unsigned i = 0; i < iters; ++i)
    if (y->operand(i).type() != op->result(i).type())
      return std::string("scf.yield operand types must match the loop results");
  return std::nullopt;
}

Diag verifyBinaryElementwise(Operation* op) {
  if (op->numOperands() != 2 || op->numResults() != 1 ||
      op->operand(0).type() != op->operand(1).type() ||
      op->operand(0).type() != op->result(0).type())
    return std::string("operands and result must have one type");
  return std::nullopt;
}

}  // namespace

std::optional<std::string> verifyOpContract(Operation* op) {
  const std::string& n = op->name;
  if (n == "frisk.kernel" || n == "func.func") return verifyKernelLike(op);
  if (n == "frisk.parallel") return verifyParallel(op);
  if (n == "frisk.gemm") return verifyGemm(op);
  if (n == "frisk.alloc_buffer") return verifyAlloc(op);
  if (n == "frisk.copy") return verifyCopy(op);
  if (n == "frisk.fill") return verifyFill(op);
  if (n == "frisk.reduce") return verifyReduce(op);
  if (n == "frisk.reduce_tensor") return verifyReduceTensor(op);
  if (n == "frisk.mma") return verifyMma(op);
  if (n == "frisk.tile_load") return verifyTileLoad(op);
  if (n == "frisk.tile_store") return verifyTileStore(op);
  if (n == "frisk.layout_view") return verifyLayoutView(op);
  if (n == "arith.constant") return verifyConstant(op);
  if (n == "scf.for") return verifyScfFor(op);
  if (n == "arith.addf" || n == "arith.maximumf" || n == "arith.minimumf" || n == "arith.mulf")
    return verifyBinaryElementwise(op);
  return std::nullopt;
}

// ============================================================================
// Whole-IR verification: structure, dominance, then each op's contract.
// ============================================================================
namespace {

// Ops whose single-block regions end in an implicit frisk.end.
bool friskImplicitTerminator(const Operation* op) {
  return op->is("frisk.kernel") || op->is("frisk.parallel") || op->is("frisk.block") ||
         op->is("frisk.for");
}

// Is `v` visible (defined before, in this or an enclosing block) at `user`?
bool dominates(Value v, Operation* user) {
  if (v.isBlockArgument()) {
    for (Block* b = user->parent; b; b = b->parentOp() ? b->parentOp()->parent : nullptr)
      if (b == v.ownerBlock()) return true;
    return false;
  }
  Operation* def = v.definingOp();
  if (!def->parent) return false;
  Operation* anc = def->parent->findAncestorOpInBlock(user);
  return anc && anc != def && def->isBeforeInBlock(anc);
}

bool verifyRec(Operation* op, std::string* diag) {
  auto fail = [&](const std::string& msg) {
    if (diag) *diag = "'" + op->name + "' op " + msg;
    return false;
  };
  for (unsigned i = 0; i < op->numOperands(); ++i)
    if (!dominates(op->operand(i), op))
      return fail("operand #" + std::to_string(i) + " does not dominate this use");
  for (auto& r : op->regions) {
    if (friskImplicitTerminator(op) && r->size() != 1)
      return fail("expects a single-block region");
    for (auto& b : r->blocks) {
      for (auto& child : b->ops) {
        if (child->isTerminator() && child.get() != b->back())
          return fail("terminator '" + child->name + "' must be the last operation in its block");
      }
      if (friskImplicitTerminator(op)) {
        Operation* t = b->terminator();
        if (!t || !t->is("frisk.end")) return fail("block must end in 'frisk.end'");
      }
      for (auto& child : b->ops)
        if (!verifyRec(child.get(), diag)) return false;
    }
  }
  if (auto msg = verifyOpContract(op)) return fail(*msg);
  return true;
}
}  // namespace

bool verify(Operation* op, std::string* diag) { return verifyRec(op, diag); }

}  // namespace fir
