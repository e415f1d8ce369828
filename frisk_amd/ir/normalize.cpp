// Legacy fragment normalization: a restatement, over this package's IR, of
// the algorithm of LegacyFragmentNormalization.cpp (Normalizer::preflight
// :227-262, process :659-706, processMath :471-555, processCopy :557-597,
// processFor :344-367, processLegacyFor :402-421, run :708-729), with the
// CDNA4 MFMA geometry check in place of the SM90 one and the gfx950 target
// in place of sm_90a.
#include "normalize.h"

#include <algorithm>
#include <map>
#include <set>

#include "layout.h"
#include "ops.h"

namespace fir {
namespace {

const char* kEscape = "legacy local fragment escapes supported normalization boundary";

struct Failure {
  std::string msg;
};

[[noreturn]] void error(Operation* op, const std::string& msg) {
  throw Failure{"'" + op->name + "' op " + msg};
}
[[noreturn]] void reject(Operation* op, const std::string& reason = "") {
  error(op, std::string(kEscape) + (reason.empty() ? "" : ": " + reason));
}

bool isLocal(Value v) {
  return v && v.type().isMemRef() && v.type().memorySpace() == MemorySpace::Local;
}

bool isSupportedRegion(const Operation* op) {
  return op->is("builtin.module") || op->is("func.func") || op->is("frisk.kernel") ||
         op->is("frisk.parallel") || op->is("scf.for") || op->is("frisk.for");
}

Operation* functionScope(Operation* op) {
  for (Operation* p = op->parentOp(); p; p = p->parentOp())
    if (p->is("func.func") || p->is("frisk.kernel")) return p;
  return nullptr;
}

Operation* parallelAncestor(Operation* op) {
  for (Operation* p = op->parentOp(); p; p = p->parentOp())
    if (p->is("frisk.parallel")) return p;
  return nullptr;
}

bool startsWith(const std::string& s, const char* p) { return s.rfind(p, 0) == 0; }

// Does `a` (no regions of interest) come before `b` in the same or an
// enclosing block?
bool properlyDominates(Operation* a, Operation* b) {
  if (!a->parent) return false;
  Operation* anc = a->parent->findAncestorOpInBlock(b);
  return anc && anc != a && a->isBeforeInBlock(anc);
}

void preorder(Operation* op, const std::function<void(Operation*)>& fn) {
  fn(op);
  for (auto& r : op->regions)
    for (auto& b : r->blocks)
      for (auto it = b->ops.begin(); it != b->ops.end();) preorder((it++)->get(), fn);
}

class Normalizer {
 public:
  explicit Normalizer(Operation* module) : module_(module), ctx_(module->ctx), b_(module->ctx) {}

  void run() {
    preflight();
    nativeAllocations();
    State state;
    process(module_->body(), state);
    for (auto it = eraseLifetimes_.rbegin(); it != eraseLifetimes_.rend(); ++it) {
      Operation* op = *it;
      for (unsigned i = 0; i < op->numResults(); ++i)
        if (!op->result(i).useEmpty()) reject(op, "residual Local uses after promotion");
      op->erase();
    }
    verifyNoLegacyLayoutIR();
  }

 private:
  using State = std::map<ValueImpl*, Value>;

  Value root(Value v) const { return (v && rootSet_.count(v.impl())) ? v : Value(); }

  Type tensorOf(Value v) { return ctx_->tensor(v.type().shape(), v.type().elementType()); }

  // ---- attribute contracts ----------------------------------------------------
  void checkAttributes(Operation* op, std::initializer_list<const char*> allowed = {}) {
    for (auto& a : op->attrs) {
      if (!startsWith(a.name, "frisk.") && a.name != "layout") continue;
      bool ok = false;
      for (const char* n : allowed) ok |= a.name == n;
      if (!ok) error(op, "legacy-attribute-contract: unsupported semantic attribute " + a.name);
    }
  }

  void verifyImportAttributes(Operation* scope, bool allowLegacyThreads) {
    static const char* allowed[] = {"frisk.target",          "frisk.legacy_semantics",
                                    "frisk.execution_threads", "frisk.execution_layout",
                                    "frisk.writer_policy",   "frisk.vector_bytes",
                                    "frisk.mma_contract",    "frisk.copy_contract",
                                    "frisk.reduction_contract"};
    preorder(scope, [&](Operation* op) {
      for (auto& a : op->attrs) {
        if (!startsWith(a.name, "frisk.")) continue;
        bool ok = std::any_of(std::begin(allowed), std::end(allowed),
                              [&](const char* n) { return a.name == n; });
        ok |= allowLegacyThreads && a.name == "frisk.threads" && op->is("frisk.gemm");
        if (!ok) error(op, "legacy-attribute-contract: unsupported semantic attribute " + a.name);
      }
    });
  }

  void verifyTensorV1(Operation* op) {
    for (Operation* c = op; c; c = c->parentOp()) {
      const bool scope = c == op || c->is("func.func") || c->is("frisk.kernel") ||
                         c->is("builtin.module");
      if (!scope) continue;
      Attribute a = c->attr("frisk.legacy_semantics");
      if (!a) continue;
      if (a.kind() == AttrKind::String && a->s == "tensor_v1") return;
      error(op, "legacy-math-contract: explicit tensor_v1 semantics required");
    }
    error(op, "legacy-math-contract: explicit tensor_v1 semantics required");
  }

  void copyMetadata(Operation* from, Operation* to) {
    for (auto& a : from->attrs)
      if (startsWith(a.name, "frisk.") && a.name != "frisk.threads" &&
          a.name != "frisk.legacy_semantics")
        to->setAttr(a.name, a.value);
  }

  // ---- preflight ----------------------------------------------------------------
  void preflight() {
    preorder(module_, [&](Operation* op) {
      if (op->is("frisk.gemm") && op->intAttr("policy") == (int64_t)GemmWarpPolicy::Auto)
        error(op, "Auto policy requires frisk.mma");
      if (op->is("frisk.gemm") || op->is("frisk.reduce")) verifyTensorV1(op);
    });
    verifyImportAttributes(module_, true);
    preorder(module_, [&](Operation* op) {
      if ((op->is("frisk.alloc_buffer") || op->is("memref.alloc")) && isLocal(op->result(0))) {
        roots_.push_back(op->result(0));
        rootSet_.insert(op->result(0).impl());
      }
    });
    for (Value r : roots_) checkLifetime(r);
    preorder(module_, [&](Operation* op) {
      if (op->is("frisk.copy") || op->is("frisk.fill") || op->is("frisk.gemm") ||
          op->is("frisk.reduce")) {
        for (auto& v : op->operands)
          if (isLocal(v) && !root(v)) reject(op, "Local operand is not a promotable allocation");
      }
      if (op->is("frisk.gemm") || op->is("frisk.reduce"))
        checkAttributes(op, {"frisk.legacy_semantics", "frisk.target", "frisk.execution_threads",
                             "frisk.threads"});
    });
  }

  void checkLifetime(Value allocation) {
    Operation* alloc = allocation.definingOp();
    Type t = allocation.type();
    Type e = t.elementType();
    if (!t.hasStaticShape() || t.layout() || t.rank() == 0 ||
        (!e.isF16() && !e.isBF16() && !e.isF32() && !e.isSignlessInteger(32)))
      reject(alloc, "Local root requires static identity f16/bf16/f32/i32 storage");
    uint64_t points = 1;
    for (int64_t x : t.shape()) {
      if (x <= 1 || (x & (x - 1)) || (uint64_t)x > 65536 / points)
        reject(alloc, "Local root requires power-of-two extents >1 and at most 65536 elements");
      points *= (uint64_t)x;
    }
    checkAttributes(alloc);
    for (Operation* p = alloc->parentOp(); p; p = p->parentOp()) {
      if (!isSupportedRegion(p)) reject(alloc, "unsupported enclosing region");
      for (auto& r : p->regions)
        if (r->size() > 1) reject(p, "general CFG is not a sequential fragment lifetime");
    }
    for (Operation* user : allocation.users()) {
      if (!user->is("frisk.fill") && !user->is("frisk.copy") && !user->is("frisk.gemm") &&
          !user->is("frisk.reduce"))
        reject(user);
      if (parallelAncestor(user) != parallelAncestor(alloc))
        reject(user, "Local root crosses a Parallel boundary");
      if (functionScope(user) != functionScope(alloc))
        reject(user, "Local root crosses a function or Kernel boundary");
      for (Operation* p = user->parentOp(); p && p != alloc->parentOp(); p = p->parentOp())
        if (!isSupportedRegion(p)) reject(user, "unsupported enclosing region");
    }
  }

  void nativeAllocations() {
    std::vector<Operation*> native;
    preorder(module_, [&](Operation* op) {
      if (op->is("frisk.alloc_buffer") && !isLocal(op->result(0))) native.push_back(op);
    });
    for (Operation* op : native) {
      Type t = op->result(0).type();
      auto space = t.memorySpace();
      if (!t.hasStaticShape() || t.layout() || !space ||
          (*space != MemorySpace::Shared && *space != MemorySpace::Global) ||
          op->intAttr("alignment") < 0)
        error(op, "legacy-storage-root: unsupported native allocation");
      checkAttributes(op);
      b_.setInsertionPoint(op);
      Operation* alloc = b_.create("memref.alloc", {}, {t});
      alloc->loc = op->loc;
      if (op->intAttr("alignment") > 0)
        alloc->setAttr("alignment", Attribute::integer(ctx_->integer(64), op->intAttr("alignment")));
      copyMetadata(op, alloc);
      op->result(0).replaceAllUsesWith(alloc->result(0));
      op->erase();
    }
  }

  // ---- values -------------------------------------------------------------------
  Value read(Value v, Operation* at, State& state) {
    Value r = root(v);
    if (!r) reject(at, "expected promotable Local fragment");
    auto it = state.find(r.impl());
    if (it == state.end() || !it->second) error(at, "legacy-fragment-uninitialized");
    return it->second;
  }

  bool storageRootOk(Value v) {
    if (v.isBlockArgument()) {
      Operation* owner = v.ownerBlock()->parentOp();
      return owner && (owner->is("frisk.kernel") || owner->is("func.func")) &&
             owner->body() == v.ownerBlock();
    }
    Operation* d = v.definingOp();
    return d->is("memref.alloc") || d->is("frisk.layout_view");
  }

  Value storageView(Value v, Operation* at) {
    if (!v.type().isMemRef() || isLocal(v) || !storageRootOk(v))
      error(at, "legacy-storage-boundary: unsupported storage alias or descriptor");
    if (!v.isBlockArgument() && v.definingOp()->is("frisk.layout_view")) return v;
    for (Operation* u : v.users())
      if (u->is("frisk.layout_view") && properlyDominates(u, at)) return u->result(0);
    b_.setInsertionPoint(at);
    Operation* view = b_.create("frisk.layout_view", {v}, {v.type()});
    view->loc = at->loc;
    return view->result(0);
  }

  std::vector<Value> modifiedExternal(Operation* scope, const State& state) {
    std::set<ValueImpl*> modified;
    scope->walk([&](Operation* op) {
      Value dst;
      if (op->is("frisk.fill")) dst = op->operand(0);
      else if (op->is("frisk.copy")) dst = op->operand(1);
      else if (op->is("frisk.gemm")) dst = op->operand(2);
      else if (op->is("frisk.reduce")) dst = op->operand(1);
      if (dst && root(dst) && state.count(root(dst).impl())) modified.insert(root(dst).impl());
    });
    std::vector<Value> ordered;
    for (Value r : roots_)
      if (modified.count(r.impl())) ordered.push_back(r);
    return ordered;
  }

  Operation* constantOp(Operation* at, Attribute value, Type t) {
    b_.setInsertionPoint(at);
    Operation* c = createConstant(b_, value, t);
    c->loc = at->loc;
    return c;
  }

  Attribute zeroSplat(Type tensor) {
    return tensor.elementType().isFloat() ? Attribute::denseFloat(tensor, {0.0})
                                          : Attribute::denseInt(tensor, {0});
  }

  int64_t threads(Operation* op, bool gemm) {
    std::optional<int64_t> expl;
    for (const char* n : {"frisk.execution_threads", "frisk.threads"}) {
      Attribute a = op->attr(n);
      if (!a) continue;
      if ((!gemm && std::string(n) == "frisk.threads") || a.kind() != AttrKind::Integer ||
          !a->type.isSignlessInteger(64) || a->i <= 0 || (expl && *expl != a->i))
        error(op, "legacy-thread-contract: malformed or conflicting execution threads");
      expl = a->i;
    }
    if (Operation* par = parallelAncestor(op)) {
      const int64_t t = par->intAttr("threads");
      if (expl && *expl != t)
        error(op, "legacy-thread-contract: execution threads conflict with Parallel");
      expl = t;
    }
    return expl.value_or(128);
  }

  // ---- rewriting ------------------------------------------------------------------
  void processMath(Operation* op, State& state) {
    const bool isGemm = op->is("frisk.gemm");
    const int64_t nthreads = threads(op, isGemm);
    if (isGemm) {
      Value A = op->operand(0), B = op->operand(1), C = op->operand(2);
      Type aT = A.type(), bT = B.type(), cT = C.type();
      Type ae = aT.elementType(), ce = cT.elementType();
      const bool intPath = ae.isSignlessInteger(8);
      if (intPath ? !ce.isSignlessInteger(32) : !ce.isF32())
        error(op, "legacy-gemm-accumulator: f32 required; implicit promotion is forbidden");
      // The reference's SM90 path takes f16/bf16 (LegacyFragmentNormalization
      // .cpp:478-494); gfx950 has MFMA atoms for fp8, i8 and f32 as well
      // (v_mfma_f32_32x32x2_f32 for an f32 product such as the reference's
      // own GEMM tile program, tmp/ir.mlir:2-16).
      const bool inOk = ae.isF16() || ae.isBF16() || ae.isF32() ||
                        ae.isFloat(FloatKind::E4M3FN) || ae.isFloat(FloatKind::E5M2) || intPath;
      if (!inOk || ae != bT.elementType())
        error(op, "legacy-gemm-input: matching f16/bf16/f32/fp8/i8 A/B required");
      if (auto err = legacyGemmValidationError(aT, bT, cT, op->boolAttr("transA"),
                                               op->boolAttr("transB"), op->intAttr("M"),
                                               op->intAttr("N"), op->intAttr("K")))
        error(op, *err);
      std::string target;
      for (Operation* s = op; s; s = s->parentOp())
        if (Attribute a = s->attr("frisk.target")) {
          if (a.kind() == AttrKind::String) target = a->s;
          break;
        }
      if (target != kCdna4Target) error(op, "cdna4-mma-target: explicit gfx950 target required");
      if (!root(C) || bT.memorySpace() != MemorySpace::Shared ||
          (!root(A) && aT.memorySpace() != MemorySpace::Shared))
        reject(op, "Gemm requires Local C, Shared B and Local/Shared A");
      Value a = root(A) ? read(A, op, state) : storageView(A, op);
      Value bv = storageView(B, op);
      Value init;
      if (op->boolAttr("clear_accum")) {
        Type t = tensorOf(C);
        init = constantOp(op, zeroSplat(t), t)->result(0);
      } else {
        init = read(C, op, state);
      }
      b_.setInsertionPoint(op);
      Type i64 = ctx_->integer(64);
      Operation* mma = b_.create("frisk.mma", {a, bv, init}, {tensorOf(C)},
                                 {{"k", Attribute::integer(i64, op->intAttr("K"))},
                                  {"m", Attribute::integer(i64, op->intAttr("M"))},
                                  {"n", Attribute::integer(i64, op->intAttr("N"))},
                                  {"policy", op->attr("policy")},
                                  {"trans_a", Attribute::boolean(op->boolAttr("transA"))},
                                  {"trans_b", Attribute::boolean(op->boolAttr("transB"))}});
      mma->loc = op->loc;
      copyMetadata(op, mma);
      mma->setAttr("frisk.execution_threads", Attribute::integer(i64, nthreads));
      if (!cdna4MmaGeometry(op->intAttr("M"), op->intAttr("N"), op->intAttr("K"), ae, ce, nthreads,
                            (GemmWarpPolicy)op->intAttr("policy")))
        error(op, "cdna4-mma-thread-group: unsupported tile, threads or policy grouping");
      state[root(C).impl()] = mma->result(0);
      op->erase();
      return;
    }
    const std::string kind = op->strAttr("kind");
    if (kind != "add" && kind != "max" && kind != "min")
      error(op, "legacy-reduce-kind: only add/max/min are supported");
    Value src = op->operand(0), dst = op->operand(1);
    if (!root(dst)) reject(op, "Reduce requires a Local destination");
    Value source;
    if (root(src)) {
      source = read(src, op, state);
    } else {
      Value view = storageView(src, op);
      b_.setInsertionPoint(op);
      Operation* load = b_.create("frisk.tile_load", {view}, {tensorOf(src)});
      load->loc = op->loc;
      source = load->result(0);
    }
    Value previous;
    if (!op->boolAttr("clear")) previous = read(dst, op, state);
    b_.setInsertionPoint(op);
    Operation* red = b_.create(
        "frisk.reduce_tensor", {source}, {tensorOf(dst)},
        {{"dim", Attribute::integer(ctx_->integer(64), op->intAttr("dim"))},
         {"kind", Attribute::string(kind == "add" ? "sum" : kind)}});
    red->loc = op->loc;
    copyMetadata(op, red);
    red->setAttr("frisk.execution_threads", Attribute::integer(ctx_->integer(64), nthreads));
    Value result = red->result(0);
    if (previous) {
      const char* merge = kind == "add" ? "arith.addf" : kind == "max" ? "arith.maximumf" : "arith.minimumf";
      Operation* m = b_.create(merge, {previous, result}, {result.type()});
      m->loc = op->loc;
      result = m->result(0);
    }
    state[root(dst).impl()] = result;
    op->erase();
  }

  void processCopy(Operation* copy, State& state) {
    CopyParts p = copyParts(copy);
    Type st = p.src.type(), dt = p.dst.type();
    if (!st.hasStaticShape() || !dt.hasStaticShape() || st.shape() != dt.shape() ||
        st.elementType() != dt.elementType() || st.shape() != p.srcExtents ||
        dt.shape() != p.dstExtents || !p.srcIdx.empty() || !p.dstIdx.empty() ||
        p.srcMap.numInputs() || p.dstMap.numInputs() || p.srcMap.numResults() ||
        p.dstMap.numResults())
      error(copy, "legacy-copy-boundary: requires static whole-tile copy with empty maps/indices");
    const bool srcLocal = (bool)root(p.src), dstLocal = (bool)root(p.dst);
    if (srcLocal || dstLocal) checkAttributes(copy);
    if (!srcLocal && !dstLocal) {
      Value s = storageView(p.src, copy), d = storageView(p.dst, copy);
      copy->setOperand(0, s);
      copy->setOperand(1, d);
      return;
    }
    Value value;
    if (srcLocal) {
      value = read(p.src, copy, state);
    } else {
      Value view = storageView(p.src, copy);
      b_.setInsertionPoint(copy);
      Operation* load = b_.create("frisk.tile_load", {view}, {tensorOf(p.src)});
      load->loc = copy->loc;
      copyMetadata(copy, load);
      value = load->result(0);
    }
    if (dstLocal) {
      state[root(p.dst).impl()] = value;
    } else {
      Value view = storageView(p.dst, copy);
      b_.setInsertionPoint(copy);
      Operation* store = b_.create("frisk.tile_store", {value, view}, {});
      store->loc = copy->loc;
      copyMetadata(copy, store);
    }
    copy->erase();
  }

  void processFor(Operation* loop, State& state) {
    std::vector<Value> modified = modifiedExternal(loop, state);
    for (Value r : modified) read(r, loop, state);
    State bodyState = state;
    if (modified.empty()) {
      process(loop->body(), bodyState);
      return;
    }
    std::vector<Value> operands = loop->operands;
    std::vector<Type> results;
    for (unsigned i = 0; i < loop->numResults(); ++i) results.push_back(loop->result(i).type());
    for (Value r : modified) {
      operands.push_back(state[r.impl()]);
      results.push_back(tensorOf(r));
    }
    b_.setInsertionPoint(loop);
    Operation* repl = b_.create("scf.for", operands, results, {}, 1);
    repl->loc = loop->loc;
    for (auto& a : loop->attrs) repl->setAttr(a.name, a.value);
    repl->region(0).takeBody(loop->region(0));
    Block* body = repl->body();
    for (Value r : modified) bodyState[r.impl()] = body->addArgument(tensorOf(r));
    process(body, bodyState);
    Operation* yield = body->terminator();
    std::vector<Value> yieldOps = yield->operands;
    for (Value r : modified) yieldOps.push_back(bodyState[r.impl()]);
    yield->setOperands(yieldOps);
    const unsigned old = loop->numResults();
    for (unsigned i = 0; i < old; ++i) loop->result(i).replaceAllUsesWith(repl->result(i));
    for (size_t i = 0; i < modified.size(); ++i)
      state[modified[i].impl()] = repl->result(old + (unsigned)i);
    loop->erase();
  }

  void processLegacyFor(Operation* loop, State& state) {
    bool touches = false;
    loop->walk([&](Operation* nested) {
      for (auto& v : nested->operands) touches |= (bool)root(v);
      for (unsigned i = 0; i < nested->numResults(); ++i) touches |= (bool)root(nested->result(i));
    });
    if (!touches) {
      process(loop->body(), state);
      return;
    }
    const int64_t lo = loop->intAttr("lower"), hi = loop->intAttr("upper"), st = loop->intAttr("step");
    if (st <= 0 || lo > hi) reject(loop, "legacy for requires a static positive-step half-open range");
    checkAttributes(loop);
    Type idx = ctx_->index();
    Value lb = constantOp(loop, Attribute::integer(idx, lo), idx)->result(0);
    Value ub = constantOp(loop, Attribute::integer(idx, hi), idx)->result(0);
    Value step = constantOp(loop, Attribute::integer(idx, st), idx)->result(0);
    b_.setInsertionPoint(loop);
    Operation* repl = b_.create("scf.for", {lb, ub, step}, {}, {}, 1);
    repl->loc = loop->loc;
    copyMetadata(loop, repl);
    repl->region(0).takeBody(loop->region(0));
    Block* body = repl->body();
    Operation* end = body->terminator();
    b_.setInsertionPoint(end);
    b_.create("scf.yield", {}, {})->loc = end->loc;
    end->erase();
    loop->erase();
    processFor(repl, state);
  }

  void processIndependentStorage(Operation* scope) {
    std::vector<Operation*> ops;
    scope->walk([&](Operation* op) { ops.push_back(op); });
    for (Operation* op : ops) {
      if (op->is("frisk.gemm") || op->is("frisk.reduce"))
        reject(op, "math import requires a supported sequential region");
      if (op->is("frisk.fill")) {
        op->setOperand(0, storageView(op->operand(0), op));
      } else if (op->is("frisk.copy")) {
        if (root(op->operand(0)) || root(op->operand(1))) reject(op);
        State none;
        processCopy(op, none);
      }
    }
  }

  void process(Block* block, State& state) {
    for (auto it = block->ops.begin(); it != block->ops.end();) {
      Operation* op = (it++)->get();
      if ((op->is("frisk.alloc_buffer") || op->is("memref.alloc")) && op->numResults() &&
          root(op->result(0))) {
        state[op->result(0).impl()] = Value();
        eraseLifetimes_.push_back(op);
      } else if (op->is("frisk.fill")) {
        Value r = root(op->operand(0));
        if (r) {
          checkAttributes(op);
          Attribute v = op->attr("value");
          Type t = tensorOf(r);
          if (!v || v.kind() != AttrKind::Float || v->type != t.elementType())
            error(op, "legacy-fill-constant: exact same-dtype floating constant required");
          Operation* c = constantOp(op, Attribute::denseFloat(t, {v->f}), t);
          copyMetadata(op, c);
          state[r.impl()] = c->result(0);
          op->erase();
        } else {
          op->setOperand(0, storageView(op->operand(0), op));
        }
      } else if (op->is("frisk.copy")) {
        processCopy(op, state);
      } else if (op->is("frisk.gemm") || op->is("frisk.reduce")) {
        processMath(op, state);
      } else if (op->is("scf.for")) {
        processFor(op, state);
      } else if (op->is("frisk.for")) {
        processLegacyFor(op, state);
      } else if (op->numRegions()) {
        if (!isSupportedRegion(op)) {
          processIndependentStorage(op);
          continue;
        }
        State nested;  // kernels, functions and parallel regions are independent scopes
        for (auto& r : op->regions) {
          if (r->empty()) continue;
          if (r->size() > 1) {
            processIndependentStorage(op);
            continue;
          }
          process(r->front(), nested);
        }
      }
    }
  }

  void verifyNoLegacyLayoutIR() {
    verifyImportAttributes(module_, false);
    preorder(module_, [&](Operation* op) {
      bool residual = op->is("frisk.alloc_buffer") || op->is("frisk.gemm") || op->is("frisk.reduce");
      if (op->is("frisk.copy") || op->is("frisk.fill"))
        for (auto& v : op->operands) residual |= isLocal(v);
      if (residual)
        error(op, "legacy layout IR requires frisk-normalize-layout-ir or frisk-layout-pipeline");
    });
  }

  Operation* module_;
  Context* ctx_;
  Builder b_;
  std::vector<Value> roots_;
  std::set<ValueImpl*> rootSet_;
  std::vector<Operation*> eraseLifetimes_;
};

}  // namespace

std::string normalizeLegacyFragments(Operation* module) {
  if (!module || !module->is("builtin.module")) return "normalization expects a builtin.module";
  try {
    Normalizer(module).run();
  } catch (const Failure& f) {
    return f.msg;
  }
  std::string diag;
  if (!verify(module, &diag)) return diag;
  return "";
}

}  // namespace fir
