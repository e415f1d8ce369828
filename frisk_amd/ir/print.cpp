// MLIR-style textual form of the tile IR.
//
// The frisk ops print in the custom assembly of the reference
// (FriskOps.cpp: kernel :136-159, parallel :207-222, block :289-304, for
// :392-401, alloc_buffer :542-547, copy :644-660; assemblyFormat of gemm,
// fill, reduce and the layout ops in FriskOps.td / FriskLayoutOps.td).
// SSA names follow MLIR's scheme: entry-block arguments `%argN`, op results
// `%N`, with `%cst`/`%c<v>`/`%alloc` names for constants and allocations.
#include <functional>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

#include "ops.h"

namespace fir {
namespace {

class AsmState {
 public:
  explicit AsmState(Operation* top) {
    if (!top) return;
    for (auto& res : top->results) names_[res.get()] = "%" + resultName(top, res.get());
    number(top);
  }

  const std::string& name(Value v) {
    auto it = names_.find(v.impl());
    if (it != names_.end()) return it->second;
    static const std::string unknown = "<<UNKNOWN SSA VALUE>>";
    return unknown;
  }

 private:
  std::string unique(const std::string& base) {
    if (!used_.count(base)) {
      used_.insert(base);
      return base;
    }
    for (int i = 0;; ++i) {
      std::string c = base + "_" + std::to_string(i);
      if (!used_.count(c)) {
        used_.insert(c);
        return c;
      }
    }
  }

  void number(Operation* op) {
    for (auto& r : op->regions) {
      bool entry = true;
      for (auto& b : r->blocks) {
        for (auto& a : b->args)
          names_[a.get()] = entry ? "%arg" + std::to_string(nextArg_++) : "%" + std::to_string(nextVal_++);
        entry = false;
        for (auto& child : b->ops) {
          for (auto& res : child->results) names_[res.get()] = "%" + resultName(child.get(), res.get());
          number(child.get());
        }
      }
    }
  }

  std::string resultName(Operation* op, ValueImpl* res) {
    if (op->is("arith.constant")) {
      Attribute v = op->attr("value");
      if (v && v.kind() == AttrKind::Integer) {
        std::string base = "c" + std::to_string(v->i);
        if (!v->type.isIndex()) base += "_" + v->type.str();
        for (char& ch : base)
          if (ch == '-') ch = 'n';
        return unique(base);
      }
      return unique("cst");
    }
    if (op->is("memref.alloc")) return unique("alloc");
    (void)res;
    return std::to_string(nextVal_++);
  }

  std::unordered_map<ValueImpl*, std::string> names_;
  std::unordered_set<std::string> used_;
  int nextArg_ = 0, nextVal_ = 0;
};

Operation* topLevel(Operation* op) {
  while (op->parentOp()) op = op->parentOp();
  return op;
}

class Printer {
 public:
  Printer(Operation* top, PrintOptions o) : st_(top), opts_(o) {}

  void op(Operation* o, int indent) {
    pad(indent);
    printResults(o);
    const std::string& n = o->name;
    if (n == "builtin.module") module(o, indent);
    else if (n == "frisk.kernel") kernel(o, indent);
    else if (n == "func.func") func(o, indent);
    else if (n == "frisk.parallel") parallel(o, indent);
    else if (n == "frisk.block") blockOp(o, indent);
    else if (n == "frisk.for") forOp(o, indent);
    else if (n == "frisk.end") os_ << "frisk.end";
    else if (n == "frisk.gemm") gemm(o);
    else if (n == "frisk.alloc_buffer") alloc(o);
    else if (n == "frisk.copy") copy(o);
    else if (n == "frisk.fill" || n == "frisk.reduce" || n == "frisk.tile_store") operandsAttrsTypes(o, {});
    else if (n == "frisk.mma") mma(o);
    else if (n == "frisk.reduce_tensor" || n == "frisk.tile_load" || n == "frisk.layout_view")
      operandsAttrsTypesArrow(o);
    else if (n == "arith.constant") constant(o);
    else if (n == "arith.addf" || n == "arith.maximumf" || n == "arith.minimumf" || n == "arith.mulf")
      binary(o);
    else if (n == "memref.alloc") memrefAlloc(o);
    else if (n == "scf.for") scfFor(o, indent);
    else if (n == "scf.yield" || n == "func.return") yield(o);
    else generic(o, indent);
    if (opts_.debugInfo) os_ << ' ' << o->loc.str();
    os_ << '\n';
  }

  std::string str() const { return os_.str(); }

  void blockOps(Block* b, int indent) {
    for (auto& child : b->ops) op(child.get(), indent);
  }

 private:
  void pad(int n) {
    for (int i = 0; i < n; ++i) os_ << "  ";
  }
  const std::string& nm(Value v) { return st_.name(v); }

  void printResults(Operation* o) {
    if (!o->numResults()) return;
    for (unsigned i = 0; i < o->numResults(); ++i) os_ << (i ? ", " : "") << nm(o->result(i));
    os_ << " = ";
  }

  void attrDict(Operation* o, std::initializer_list<const char*> elide, bool keyword = false) {
    std::vector<const NamedAttr*> shown;
    for (auto& a : o->attrs) {
      bool skip = false;
      for (const char* e : elide) skip |= a.name == e;
      if (!skip) shown.push_back(&a);
    }
    if (shown.empty()) return;
    os_ << (keyword ? " attributes {" : " {");
    for (size_t i = 0; i < shown.size(); ++i) {
      os_ << (i ? ", " : "") << shown[i]->name;
      if (shown[i]->value.kind() != AttrKind::Unit) os_ << " = " << shown[i]->value.str();
    }
    os_ << '}';
  }

  void operandList(Operation* o, unsigned from = 0, unsigned to = ~0u) {
    to = std::min(to, o->numOperands());
    for (unsigned i = from; i < to; ++i) os_ << (i > from ? ", " : "") << nm(o->operand(i));
  }

  void typeList(const std::vector<Type>& ts) {
    for (size_t i = 0; i < ts.size(); ++i) os_ << (i ? ", " : "") << ts[i].str();
  }

  std::vector<Type> operandTypes(Operation* o) {
    std::vector<Type> ts;
    for (auto& v : o->operands) ts.push_back(v.type());
    return ts;
  }

  // Print the blocks of a region.  The entry block's header is printed only
  // when asked for and it has arguments; non-entry blocks always get one.
  void region(Region& r, int indent, bool entryArgs, bool terminators) {
    os_ << "{\n";
    bool entry = true;
    int label = 0;
    for (auto& b : r.blocks) {
      if (!entry || (entryArgs && b->numArguments())) {
        pad(indent);
        os_ << "^bb" << label;
        if (b->numArguments()) {
          os_ << '(';
          for (unsigned i = 0; i < b->numArguments(); ++i)
            os_ << (i ? ", " : "") << nm(b->argument(i)) << ": " << b->argument(i).type().str();
          os_ << ')';
        }
        os_ << ":\n";
      }
      ++label;
      for (auto& child : b->ops) {
        if (!terminators && child.get() == b->back() && child->isTerminator() &&
            child->numOperands() == 0)
          continue;
        op(child.get(), indent + 1);
      }
      entry = false;
    }
    pad(indent);
    os_ << '}';
  }

  void module(Operation* o, int indent) {
    os_ << "module";
    attrDict(o, {"sym_name"}, true);
    os_ << ' ';
    region(o->region(0), indent, false, true);
  }

  void kernel(Operation* o, int indent) {
    os_ << "frisk.kernel @" << o->strAttr("sym_name") << '(';
    Type ft = o->attr("function_type")->type;
    typeList(ft.inputs());
    os_ << ')';
    if (!ft.results().empty()) {
      os_ << " -> (";
      typeList(ft.results());
      os_ << ')';
    }
    os_ << ' ';
    region(o->region(0), indent, true, true);
    attrDict(o, {"sym_name", "function_type"});
  }

  void func(Operation* o, int indent) {
    os_ << "func.func @" << o->strAttr("sym_name") << '(';
    Type ft = o->attr("function_type")->type;
    Block* body = o->body();
    auto ins = ft.inputs();
    for (size_t i = 0; i < ins.size(); ++i) {
      os_ << (i ? ", " : "");
      if (body) os_ << nm(body->argument((unsigned)i)) << ": ";
      os_ << ins[i].str();
    }
    os_ << ')';
    auto outs = ft.results();
    if (!outs.empty()) {
      os_ << " -> ";
      if (outs.size() > 1) os_ << '(';
      typeList(outs);
      if (outs.size() > 1) os_ << ')';
    }
    attrDict(o, {"sym_name", "function_type"}, true);
    if (body) {
      os_ << ' ';
      region(o->region(0), indent, false, true);
    }
  }

  void ivs(Block* b) {
    os_ << '(';
    if (b)
      for (unsigned i = 0; i < b->numArguments(); ++i) os_ << (i ? ", " : "") << nm(b->argument(i));
    os_ << ')';
  }

  void i64s(const std::vector<int64_t>& v) {
    for (size_t i = 0; i < v.size(); ++i) os_ << (i ? ", " : "") << v[i];
  }

  void parallel(Operation* o, int indent) {
    os_ << "frisk.parallel ";
    ivs(o->body());
    os_ << " = (";
    i64s(i64Array(o, "ranges"));
    os_ << "), threads = " << o->intAttr("threads") << ' ';
    region(o->region(0), indent, false, true);
  }

  void blockOp(Operation* o, int indent) {
    os_ << "frisk.block ";
    ivs(o->body());
    os_ << " to (";
    i64s(i64Array(o, "ranges"));
    os_ << ") ";
    region(o->region(0), indent, false, false);
  }

  void forOp(Operation* o, int indent) {
    os_ << "frisk.for ";
    Block* b = o->body();
    os_ << (b && b->numArguments() ? nm(b->argument(0)) : std::string("%?")) << " = "
        << o->intAttr("lower") << " to " << o->intAttr("upper");
    if (o->intAttr("step") > 1) os_ << " step = " << o->intAttr("step");
    os_ << ' ';
    region(o->region(0), indent, false, false);
  }

  void gemm(Operation* o) {
    os_ << "frisk.gemm(";
    operandList(o);
    os_ << ')';
    attrDict(o, {});
    os_ << " : ";
    typeList(operandTypes(o));
  }

  void alloc(Operation* o) {
    os_ << "frisk.alloc_buffer";
    attrDict(o, {"shape", "elementType", "memorySpace"});
    os_ << " -> " << o->result(0).type().str();
  }

  // `%x[<map results with dims replaced by the index operands>]`.
  void mapOfSsaIds(AffineMap map, const std::vector<Value>& idx) {
    std::vector<std::string> names;
    for (auto& v : idx) names.push_back(nm(v));
    for (unsigned r = 0; r < map.numResults(); ++r) {
      os_ << (r ? ", " : "");
      std::function<void(AffineExpr, bool)> pe = [&](AffineExpr e, bool strong) {
        switch (e.kind()) {
          case AffineKind::DimId:
            os_ << (e.position() < names.size() ? names[e.position()] : "d" + std::to_string(e.position()));
            return;
          case AffineKind::SymbolId: {
            unsigned p = map.numDims() + e.position();
            os_ << "symbol(" << (p < names.size() ? names[p] : "s" + std::to_string(e.position())) << ')';
            return;
          }
          case AffineKind::Constant: os_ << e.value(); return;
          default: break;
        }
        if (strong) os_ << '(';
        const char* opn = e.kind() == AffineKind::Add ? " + " : e.kind() == AffineKind::Mul ? " * "
                          : e.kind() == AffineKind::Mod ? " mod "
                          : e.kind() == AffineKind::FloorDiv ? " floordiv " : " ceildiv ";
        pe(e.lhs(), e.kind() != AffineKind::Add);
        os_ << opn;
        pe(e.rhs(), e.kind() != AffineKind::Add);
        if (strong) os_ << ')';
      };
      pe(map.result(r), false);
    }
  }

  void copy(Operation* o) {
    CopyParts p = copyParts(o);
    os_ << "frisk.copy " << nm(p.src) << '[';
    mapOfSsaIds(p.srcMap, p.srcIdx);
    os_ << "], " << nm(p.dst) << '[';
    mapOfSsaIds(p.dstMap, p.dstIdx);
    os_ << ']';
    attrDict(o, {"srcMap", "dstMap", "operandSegmentSizes"});
    os_ << " : " << p.src.type().str() << ", " << p.dst.type().str();
  }

  void operandsAttrsTypes(Operation* o, std::initializer_list<const char*> elide) {
    os_ << o->name << ' ';
    operandList(o);
    attrDict(o, elide);
    os_ << " : ";
    typeList(operandTypes(o));
  }

  // Generated assembly formats elide attributes equal to their declared
  // default (trans_a = trans_b = false, policy = Square; FriskLayoutOps.td).
  void mma(Operation* o) {
    std::vector<const char*> elide;
    Attribute ta = o->attr("trans_a"), tb = o->attr("trans_b"), pol = o->attr("policy");
    if (ta && ta.kind() == AttrKind::Bool && !ta->b) elide.push_back("trans_a");
    if (tb && tb.kind() == AttrKind::Bool && !tb->b) elide.push_back("trans_b");
    if (pol && pol.kind() == AttrKind::GemmPolicyA && pol->i == 0) elide.push_back("policy");
    os_ << o->name << ' ';
    operandList(o);
    attrDictElide(o, elide);
    os_ << " : ";
    typeList(operandTypes(o));
    os_ << " -> " << o->result(0).type().str();
  }

  void attrDictElide(Operation* o, const std::vector<const char*>& elide) {
    bool first = true;
    for (auto& a : o->attrs) {
      bool skip = false;
      for (const char* e : elide) skip |= a.name == e;
      if (skip) continue;
      os_ << (first ? " {" : ", ") << a.name;
      if (a.value.kind() != AttrKind::Unit) os_ << " = " << a.value.str();
      first = false;
    }
    if (!first) os_ << '}';
  }

  void operandsAttrsTypesArrow(Operation* o) {
    operandsAttrsTypes(o, {});
    os_ << " -> " << o->result(0).type().str();
  }

  void constant(Operation* o) {
    os_ << "arith.constant ";
    Attribute v = o->attr("value");
    if (v.kind() == AttrKind::DenseFloat || v.kind() == AttrKind::DenseInt) {
      os_ << v.str();
    } else if (v.kind() == AttrKind::Integer && v->type.isIndex()) {
      os_ << v->i << " : index";
    } else {
      os_ << v.str();
    }
    attrDict(o, {"value"});
  }

  void binary(Operation* o) {
    os_ << o->name << ' ';
    operandList(o);
    attrDict(o, {});
    os_ << " : " << o->result(0).type().str();
  }

  void memrefAlloc(Operation* o) {
    os_ << "memref.alloc(";
    operandList(o);
    os_ << ')';
    attrDict(o, {});
    os_ << " : " << o->result(0).type().str();
  }

  void scfFor(Operation* o, int indent) {
    Block* b = o->body();
    os_ << "scf.for " << nm(b->argument(0)) << " = " << nm(o->operand(0)) << " to "
        << nm(o->operand(1)) << " step " << nm(o->operand(2));
    if (o->numOperands() > 3) {
      os_ << " iter_args(";
      for (unsigned i = 3; i < o->numOperands(); ++i)
        os_ << (i > 3 ? ", " : "") << nm(b->argument(i - 2)) << " = " << nm(o->operand(i));
      os_ << ") -> (";
      std::vector<Type> rt;
      for (unsigned i = 0; i < o->numResults(); ++i) rt.push_back(o->result(i).type());
      typeList(rt);
      os_ << ')';
    }
    attrDict(o, {});
    os_ << ' ';
    region(o->region(0), indent, false, false);
  }

  void yield(Operation* o) {
    os_ << (o->is("func.return") ? "return" : o->name.c_str());
    if (o->numOperands()) {
      os_ << ' ';
      operandList(o);
      os_ << " : ";
      typeList(operandTypes(o));
    }
    attrDict(o, {});
  }

  void generic(Operation* o, int indent) {
    os_ << '"' << o->name << "\"(";
    operandList(o);
    os_ << ')';
    if (o->numRegions()) {
      os_ << " (";
      for (unsigned i = 0; i < o->numRegions(); ++i) {
        if (i) os_ << ", ";
        region(o->region(i), indent, true, true);
      }
      os_ << ')';
    }
    attrDict(o, {});
    os_ << " : (";
    typeList(operandTypes(o));
    os_ << ") -> (";
    std::vector<Type> rt;
    for (unsigned i = 0; i < o->numResults(); ++i) rt.push_back(o->result(i).type());
    typeList(rt);
    os_ << ')';
  }

  AsmState st_;
  PrintOptions opts_;
  std::ostringstream os_;
};

}  // namespace

std::string printOp(Operation* op, PrintOptions opts) {
  Printer p(topLevel(op), opts);
  p.op(op, 0);
  std::string s = p.str();
  if (!s.empty() && s.back() == '\n') s.pop_back();
  return s;
}

std::string printBlock(Block* b, PrintOptions opts) {
  Operation* parent = b->parentOp();
  Printer p(parent ? topLevel(parent) : nullptr, opts);
  p.blockOps(b, 0);
  std::string s = p.str();
  if (!s.empty() && s.back() == '\n') s.pop_back();
  return s;
}

std::string printValueAsOperand(Value v) {
  Operation* anchor = v.isBlockArgument() ? v.ownerBlock()->parentOp() : v.definingOp();
  if (!anchor) return "<<UNKNOWN SSA VALUE>>";
  AsmState st(topLevel(anchor));
  return st.name(v);
}

}  // namespace fir
