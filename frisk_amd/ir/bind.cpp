// Python module `frisk_ffi` (submodules `ir` and `ir.frisk`): the IR builder
// surface of the reference's pybind11 module (ffi/ir.cpp, ffi/ffi.cpp) with
// the same class, method and argument names, over the host tile IR of this
// package.  Contract violations raise ValueError (std::invalid_argument) and
// out-of-range indices IndexError, as in the reference.
//
// Lifetimes follow the reference: the `context` object owns everything built
// in it; handles returned here (operations, blocks, regions, values) are
// non-owning and must not outlive the context.  `builder` keeps its context
// alive, and `module` accepts a `.context` attribute for the same purpose
// (utils.py:55-56 in the reference).
#include <pybind11/functional.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <iostream>
#include <map>
#include <numeric>

#include "layout.h"
#include "infer.h"
#include "parse.h"
#include "normalize.h"
#include "ops.h"

namespace py = pybind11;
using namespace fir;

namespace {

// ---- wrappers ---------------------------------------------------------------
struct PyType { Type t; };
struct PyTensorType : PyType {};
struct PyMemRefType : PyType {};
struct PyFunctionType : PyType {};

struct PyValue { Value v; };
struct PyOpResult : PyValue {};
struct PyBlockArgument : PyValue {};
struct PyValueRange { std::vector<Value> vals; };

struct PyAttr { Attribute a; };
struct PyIntegerAttr : PyAttr {};
struct PyBoolAttr : PyAttr {};

struct PyLocation { Location l; };
struct PyInsertPoint { InsertPoint ip; };

struct PyOpState { Operation* op; };
struct PyModule : PyOpState {};
struct PyFunc : PyOpState {};
struct PyConstant : PyOpState {};
struct PyGemmOp : PyOpState {};
struct PyKernelOp : PyOpState {};
struct PyParallelOp : PyOpState {};
struct PyBlockOp : PyOpState {};
struct PyForOp : PyOpState {};
struct PyAllocBufferOp : PyOpState {};
struct PyCopyOp : PyOpState {};
struct PyFillOp : PyOpState {};
struct PyReduceOp : PyOpState {};

struct AffineBinaryOpExprW : AffineExpr { using AffineExpr::AffineExpr; };
struct AffineDimExprW : AffineExpr { using AffineExpr::AffineExpr; };
struct AffineSymbolExprW : AffineExpr { using AffineExpr::AffineExpr; };
struct AffineConstantExprW : AffineExpr { using AffineExpr::AffineExpr; };

struct PyBuilder {
  explicit PyBuilder(Context* c) : b(c) {}
  Builder b;
};

py::object wrapType(Type t) {
  if (!t) return py::none();
  if (t.isMemRef()) return py::cast(PyMemRefType{{t}});
  if (t.isTensor()) return py::cast(PyTensorType{{t}});
  if (t.isFunction()) return py::cast(PyFunctionType{{t}});
  return py::cast(PyType{t});
}

py::object wrapValue(Value v) {
  if (!v) return py::none();
  if (v.isBlockArgument()) return py::cast(PyBlockArgument{{v}});
  return py::cast(PyOpResult{{v}});
}

py::list wrapValues(const std::vector<Value>& vs) {
  py::list l;
  for (auto& v : vs) l.append(wrapValue(v));
  return l;
}

std::vector<Value> unwrapValues(const std::vector<PyValue>& vs) {
  std::vector<Value> out;
  for (auto& v : vs) out.push_back(v.v);
  return out;
}

std::vector<Type> unwrapTypes(const std::vector<PyType>& ts) {
  std::vector<Type> out;
  for (auto& t : ts) out.push_back(t.t);
  return out;
}

Operation* requireOp(const PyOpState& s) {
  if (!s.op) throw InvalidArgument("operation handle is null");
  return s.op;
}

std::string verifyMessage(Operation* op) {
  std::string diag;
  if (verify(op, &diag)) return "";
  return diag.empty() ? std::string("verification failed") : diag;
}

void emitToStderr(const std::string& s) {
  py::module_::import("sys").attr("stderr").attr("write")(s + "\n");
}

Location currentLoc(PyBuilder& b) { return b.b.loc(); }

// Python value of an attribute (introspection helper of execute()).
py::object attrToPython(const Attribute& a) {
  if (!a) return py::none();
  switch (a.kind()) {
    case AttrKind::Unit: return py::bool_(true);
    case AttrKind::Bool: return py::bool_(a->b);
    case AttrKind::Integer: return py::int_(a->i);
    case AttrKind::Float: return py::float_(a->f);
    case AttrKind::String: case AttrKind::Opaque: return py::str(a->s);
    case AttrKind::TypeA: return wrapType(a->type);
    case AttrKind::DenseI64Array: return py::cast(a->ints);
    case AttrKind::AffineMapA: return py::cast(a->map);
    case AttrKind::MemorySpaceA: return py::cast((MemorySpace)a->i);
    case AttrKind::GemmPolicyA: return py::cast((GemmWarpPolicy)a->i);
    case AttrKind::DenseFloat: return py::cast(a->floats);
    case AttrKind::DenseInt: return py::cast(a->ints);
  }
  return py::none();
}

// Whole-structure dtype names of the builder (ffi/ir.cpp:164-176).
Type floatAttrType(Context* ctx, const std::string& dtype) {
  Type t = dtypeToType(ctx, dtype);
  if (!t.isFloat()) throw InvalidArgument("invalid float type");
  return t;
}

template <class T>
py::object opAs(Operation* op, const char* name) {
  if (!op || op->name != name) return py::none();
  return py::cast(T{{op}});
}

// Python callbacks of create_block_op / create_for_op: log and rethrow
// (ffi/ir.cpp:371-394).
template <class F>
void runCallback(const char* what, F&& f) {
  try {
    f();
  } catch (py::error_already_set& e) {
    std::cerr << "Python exception in frisk " << what << ": " << e.what() << "\n";
    throw;
  }
}

// Simplification of a pure affine expression by flattening it into
// c0*d0 + ... + cs*s_s + c (mlir::simplifyAffineExpr restricted to the
// div/mod-free case); other expressions are rebuilt from simplified parts.
bool flatten(AffineExpr e, unsigned nd, unsigned ns, std::vector<int64_t>& coef) {
  switch (e.kind()) {
    case AffineKind::Constant: coef.back() += e.value(); return true;
    case AffineKind::DimId: if (e.position() >= nd) return false; coef[e.position()] += 1; return true;
    case AffineKind::SymbolId: if (e.position() >= ns) return false; coef[nd + e.position()] += 1; return true;
    case AffineKind::Add: return flatten(e.lhs(), nd, ns, coef) && flatten(e.rhs(), nd, ns, coef);
    case AffineKind::Mul: {
      AffineExpr l = e.lhs(), r = e.rhs();
      if (r.kind() != AffineKind::Constant) std::swap(l, r);
      if (r.kind() != AffineKind::Constant) return false;
      std::vector<int64_t> sub(coef.size(), 0);
      if (!flatten(l, nd, ns, sub)) return false;
      for (size_t i = 0; i < coef.size(); ++i) coef[i] += sub[i] * r.value();
      return true;
    }
    default: return false;
  }
}

AffineExpr simplifyExpr(AffineExpr e, unsigned nd, unsigned ns) {
  std::vector<int64_t> coef(nd + ns + 1, 0);
  Context* c = e.context();
  if (flatten(e, nd, ns, coef)) {
    AffineExpr r = getAffineConstantExpr(0, c);
    for (unsigned i = 0; i < nd; ++i)
      if (coef[i]) r = r + getAffineDimExpr(i, c) * coef[i];
    for (unsigned i = 0; i < ns; ++i)
      if (coef[nd + i]) r = r + getAffineSymbolExpr(i, c) * coef[nd + i];
    return r + coef.back();
  }
  if (!e.isBinary()) return e;
  return getAffineBinaryOpExpr(e.kind(), simplifyExpr(e.lhs(), nd, ns), simplifyExpr(e.rhs(), nd, ns));
}

void bindAffine(py::module_& m) {
  py::enum_<AffineKind>(m, "AffineExprKind", py::module_local())
      .value("Add", AffineKind::Add)
      .value("Mul", AffineKind::Mul)
      .value("Mod", AffineKind::Mod)
      .value("FloorDiv", AffineKind::FloorDiv)
      .value("CeilDiv", AffineKind::CeilDiv)
      .value("LAST_AFFINE_BINARY_OP", AffineKind::CeilDiv)
      .value("Constant", AffineKind::Constant)
      .value("DimId", AffineKind::DimId)
      .value("SymbolId", AffineKind::SymbolId);

  py::class_<AffineMap>(m, "AffineMap", py::module_local())
      .def(py::init<>())
      .def_static("get", [](Context* c) { return AffineMap::get(c); })
      .def_static("get", [](unsigned d, unsigned s, Context* c) { return AffineMap::get(d, s, c); })
      .def_static("get", [](unsigned d, unsigned s, AffineExpr r) { return AffineMap::get(d, s, r); })
      .def_static("get", [](unsigned d, unsigned s, std::vector<AffineExpr> r, Context* c) {
        return AffineMap::get(d, s, r, c);
      })
      .def_static("get_constant_map", [](int64_t v, Context* c) { return AffineMap::constantMap(v, c); })
      .def_static("get_multi_dim_identity_map",
                  [](unsigned n, Context* c) { return AffineMap::multiDimIdentity(n, c); })
      .def_static("get_minor_identity_map", [](unsigned d, unsigned r, Context* c) {
        return AffineMap::minorIdentity(d, r, c);
      })
      .def_static("get_permutation_map", [](std::vector<int64_t> p, Context* c) {
        std::vector<unsigned> u;
        for (int64_t x : p) {
          if (x < 0) throw InvalidArgument("not a permutation");
          u.push_back((unsigned)x);
        }
        return AffineMap::permutation(u, c);
      })
      .def_static("get_multi_dim_map_with_targets",
                  [](unsigned n, Context* c) { return AffineMap::multiDimIdentity(n, c); })
      .def("__eq__", [](const AffineMap& a, const AffineMap& b) { return a == b; })
      .def("__ne__", [](const AffineMap& a, const AffineMap& b) { return a != b; })
      .def("__hash__", [](const AffineMap& a) { return std::hash<const void*>()(a.impl()); })
      .def("__bool__", [](const AffineMap& a) { return (bool)a; })
      .def("__nonzero__", [](const AffineMap& a) { return (bool)a; })
      .def("__str__", &AffineMap::str)
      .def("__repr__", [](const AffineMap& a) { return "AffineMap(" + a.str() + ")"; })
      .def("get_num_dims", &AffineMap::numDims)
      .def("get_num_symbols", &AffineMap::numSymbols)
      .def("get_num_results", &AffineMap::numResults)
      .def("get_num_inputs", &AffineMap::numInputs)
      .def("get_results", [](const AffineMap& a) { return a.results(); })
      .def("get_result", [](const AffineMap& a, unsigned i) {
        if (i >= a.numResults()) throw py::index_error("AffineMap result index out of range");
        return a.result(i);
      })
      .def("is_identity", &AffineMap::isIdentity)
      .def("is_symbol_identity", &AffineMap::isSymbolIdentity)
      .def("is_minor_identity", &AffineMap::isMinorIdentity)
      .def("is_empty", &AffineMap::isEmpty)
      .def("is_single_constant", &AffineMap::isSingleConstant)
      .def("is_constant", &AffineMap::isConstant)
      .def("is_permutation", &AffineMap::isPermutation)
      .def("is_projected_permutation", &AffineMap::isProjectedPermutation,
           py::arg("allow_zero_in_results") = false)
      .def("get_single_constant_result", &AffineMap::singleConstantResult)
      .def("get_constant_results", &AffineMap::constantResults)
      .def("get_dim_position", &AffineMap::dimPosition, py::arg("idx"))
      .def("get_result_position", [](const AffineMap& a, AffineExpr e) -> py::object {
        auto r = a.resultPosition(e);
        if (!r) return py::none();
        return py::cast(*r);
      })
      .def("evaluate", [](const AffineMap& a, std::vector<int64_t> d, std::vector<int64_t> s) {
        return a.eval(d, s);
      }, py::arg("dims"), py::arg("symbols") = std::vector<int64_t>{});

  py::class_<AffineExpr>(m, "AffineExpr", py::module_local())
      .def(py::init<>())
      .def("__eq__", [](const AffineExpr& a, const AffineExpr& b) { return a == b; })
      .def("__eq__", [](const AffineExpr& a, int64_t v) { return a == v; })
      .def("__ne__", [](const AffineExpr& a, const AffineExpr& b) { return a != b; })
      .def("__ne__", [](const AffineExpr& a, int64_t v) { return !(a == v); })
      .def("__hash__", [](const AffineExpr& a) { return std::hash<const void*>()(a.impl()); })
      .def("__bool__", [](const AffineExpr& a) { return (bool)a; })
      .def("__nonzero__", [](const AffineExpr& a) { return (bool)a; })
      .def("__str__", &AffineExpr::str)
      .def("__repr__", [](const AffineExpr& a) { return "AffineExpr(" + a.str() + ")"; })
      .def("get_context", &AffineExpr::context, py::return_value_policy::reference)
      .def("get_kind", &AffineExpr::kind)
      .def("is_symbolic_or_constant", &AffineExpr::isSymbolicOrConstant)
      .def("is_pure_affine", &AffineExpr::isPureAffine)
      .def("get_largest_known_divisor", &AffineExpr::largestKnownDivisor)
      .def("is_multiple_of", &AffineExpr::isMultipleOf)
      .def("is_function_of_dim", &AffineExpr::isFunctionOfDim)
      .def("is_function_of_symbol", &AffineExpr::isFunctionOfSymbol)
      .def("replace_dims_and_symbols", &AffineExpr::replaceDimsAndSymbols)
      .def("replace_dims", [](const AffineExpr& a, std::vector<AffineExpr> d) {
        return a.replaceDimsAndSymbols(d, {});
      })
      .def("replace_symbols", [](const AffineExpr& a, std::vector<AffineExpr> s) {
        return a.replaceDimsAndSymbols({}, s);
      })
      .def("replace", [](const AffineExpr& a, AffineExpr target, AffineExpr repl) {
        return a.replace({{target.impl(), repl}});
      })
      .def("replace_with_map", [](const AffineExpr& a, py::dict d) {
        std::map<const AffineExprStorage*, AffineExpr> m;
        for (auto item : d) m[item.first.cast<AffineExpr>().impl()] = item.second.cast<AffineExpr>();
        return a.replace(m);
      })
      .def("shift_dims", &AffineExpr::shiftDims, py::arg("num_dims"), py::arg("shift"),
           py::arg("offset") = 0)
      .def("shift_symbols", &AffineExpr::shiftSymbols, py::arg("num_symbols"), py::arg("shift"),
           py::arg("offset") = 0)
      .def("__add__", [](const AffineExpr& a, int64_t v) { return a + v; })
      .def("__add__", [](const AffineExpr& a, const AffineExpr& b) { return a + b; })
      .def("__radd__", [](const AffineExpr& a, int64_t v) { return a + v; })
      .def("__neg__", [](const AffineExpr& a) { return -a; })
      .def("__sub__", [](const AffineExpr& a, int64_t v) { return a - v; })
      .def("__sub__", [](const AffineExpr& a, const AffineExpr& b) { return a - b; })
      .def("__rsub__", [](const AffineExpr& a, int64_t v) {
        return getAffineConstantExpr(v, a.context()) - a;
      })
      .def("__mul__", [](const AffineExpr& a, int64_t v) { return a * v; })
      .def("__mul__", [](const AffineExpr& a, const AffineExpr& b) { return a * b; })
      .def("__rmul__", [](const AffineExpr& a, int64_t v) { return a * v; })
      .def("floor_div", [](const AffineExpr& a, uint64_t v) { return floorDiv(a, v); })
      .def("floor_div", [](const AffineExpr& a, const AffineExpr& b) { return floorDiv(a, b); })
      .def("ceil_div", [](const AffineExpr& a, uint64_t v) { return ceilDiv(a, v); })
      .def("ceil_div", [](const AffineExpr& a, const AffineExpr& b) { return ceilDiv(a, b); })
      .def("__mod__", [](const AffineExpr& a, uint64_t v) { return a % v; })
      .def("__mod__", [](const AffineExpr& a, const AffineExpr& b) { return a % b; })
      .def("compose", [](const AffineExpr& a, const AffineMap& map) {
        return a.replaceDimsAndSymbols(map.results(), {});
      })
      .def("evaluate", [](const AffineExpr& a, std::vector<int64_t> d, std::vector<int64_t> s) {
        return a.eval(d, s);
      }, py::arg("dims"), py::arg("symbols") = std::vector<int64_t>{})
      .def("as_binary", [](const AffineExpr& a) -> py::object {
        if (!a.isBinary()) return py::none();
        return py::cast(AffineBinaryOpExprW(a.impl()));
      })
      .def("as_dim", [](const AffineExpr& a) -> py::object {
        if (a.kind() != AffineKind::DimId) return py::none();
        return py::cast(AffineDimExprW(a.impl()));
      })
      .def("as_symbol", [](const AffineExpr& a) -> py::object {
        if (a.kind() != AffineKind::SymbolId) return py::none();
        return py::cast(AffineSymbolExprW(a.impl()));
      })
      .def("as_constant", [](const AffineExpr& a) -> py::object {
        if (a.kind() != AffineKind::Constant) return py::none();
        return py::cast(AffineConstantExprW(a.impl()));
      });

  py::class_<AffineBinaryOpExprW, AffineExpr>(m, "AffineBinaryOpExpr", py::module_local())
      .def("get_lhs", [](const AffineBinaryOpExprW& e) { return e.lhs(); })
      .def("get_rhs", [](const AffineBinaryOpExprW& e) { return e.rhs(); });
  py::class_<AffineDimExprW, AffineExpr>(m, "AffineDimExpr", py::module_local())
      .def("get_position", [](const AffineDimExprW& e) { return e.position(); });
  py::class_<AffineSymbolExprW, AffineExpr>(m, "AffineSymbolExpr", py::module_local())
      .def("get_position", [](const AffineSymbolExprW& e) { return e.position(); });
  py::class_<AffineConstantExprW, AffineExpr>(m, "AffineConstantExpr", py::module_local())
      .def("get_value", [](const AffineConstantExprW& e) { return e.value(); });

  m.def("get_affine_dim_expr", &getAffineDimExpr);
  m.def("get_affine_symbol_expr", &getAffineSymbolExpr);
  m.def("get_affine_constant_expr", &getAffineConstantExpr);
  m.def("get_affine_constant_exprs", [](std::vector<int64_t> vs, Context* c) {
    std::vector<AffineExpr> out;
    for (int64_t v : vs) out.push_back(getAffineConstantExpr(v, c));
    return out;
  });
  m.def("get_affine_binary_op_expr", &getAffineBinaryOpExpr);
  // Flat form [dims..., symbols..., locals..., constant] (mlir::getAffineExprFromFlatForm).
  m.def("get_affine_expr_from_flat_form", [](std::vector<int64_t> flat, unsigned nd, unsigned ns,
                                              std::vector<AffineExpr> locals, Context* c) {
    if (flat.size() != nd + ns + locals.size() + 1)
      throw InvalidArgument("flat form needs dims + symbols + locals + 1 coefficients");
    AffineExpr r = getAffineConstantExpr(0, c);
    for (unsigned i = 0; i < nd; ++i)
      if (flat[i]) r = r + getAffineDimExpr(i, c) * flat[i];
    for (unsigned i = 0; i < ns; ++i)
      if (flat[nd + i]) r = r + getAffineSymbolExpr(i, c) * flat[nd + i];
    for (size_t i = 0; i < locals.size(); ++i)
      if (flat[nd + ns + i]) r = r + locals[i] * flat[nd + ns + i];
    return r + flat.back();
  });
  m.def("simplify_affine_expr", &simplifyExpr);
}

// ---- core classes -------------------------------------------------------------
void bindCore(py::module_& m) {
  py::class_<Context>(m, "context", py::module_local())
      .def(py::init<>())
      .def("disable_multithreading", &Context::disableMultithreading);

  py::enum_<MemorySpace>(m, "MemorySpace", py::arithmetic())
      .value("GLOBAL", MemorySpace::Global)
      .value("SHARED", MemorySpace::Shared)
      .value("LOCAL", MemorySpace::Local);
  py::enum_<GemmWarpPolicy>(m, "GemmWarpPolicy", py::arithmetic())
      .value("Square", GemmWarpPolicy::Square)
      .value("FullRow", GemmWarpPolicy::FullRow)
      .value("FullCol", GemmWarpPolicy::FullCol)
      .value("Auto", GemmWarpPolicy::Auto);

  py::class_<PyType>(m, "type", py::module_local())
      .def("__str__", [](const PyType& t) { return t.t.str(); })
      .def("__repr__", [](const PyType& t) { return t.t.str(); })
      .def("__eq__", [](const PyType& a, const PyType& b) { return a.t == b.t; })
      .def("__hash__", [](const PyType& a) { return std::hash<const void*>()(a.t.impl()); })
      .def("to_ranked_tensor_ty", [](const PyType& t) -> py::object {
        if (!t.t.isTensor()) return py::none();
        return py::cast(PyTensorType{{t.t}});
      })
      .def("is_f16", [](const PyType& t) { return t.t.isF16(); })
      .def("is_bf16", [](const PyType& t) { return t.t.isBF16(); })
      .def("is_f32", [](const PyType& t) { return t.t.isF32(); })
      .def("is_f64", [](const PyType& t) { return t.t.isF64(); })
      .def("is_float", [](const PyType& t) { return t.t.isFloat(); })
      .def("is_index", [](const PyType& t) { return t.t.isIndex(); })
      .def("is_int", [](const PyType& t) { return t.t.isInteger(); })
      .def("is_signed_int", [](const PyType& t) { return t.t.isSignedInteger(); })
      .def("is_unsigned_int", [](const PyType& t) { return t.t.isUnsignedInteger(); })
      .def("is_signless_int", [](const PyType& t) { return t.t.isSignlessInteger(); });

  py::class_<PyTensorType, PyType>(m, "ranked_tensor", py::module_local())
      .def("get_rank", [](const PyTensorType& t) { return t.t.rank(); })
      .def("get_shape", [](const PyTensorType& t) { return t.t.shape(); })
      .def("get_element_ty", [](const PyTensorType& t) { return wrapType(t.t.elementType()); });

  py::class_<PyMemRefType, PyType>(m, "memref_buffer", py::module_local())
      .def("get_rank", [](const PyMemRefType& t) { return t.t.rank(); })
      .def("get_dim_size", [](const PyMemRefType& t, int64_t i) {
        if (i < 0 || i >= t.t.rank()) throw py::index_error("memref dimension out of range");
        return t.t.dim(i);
      })
      .def("get_elem_width", [](const PyMemRefType& t) { return t.t.elementType().bitWidth(); })
      .def("get_shape", [](const PyMemRefType& t) { return t.t.shape(); })
      .def("get_element_ty", [](const PyMemRefType& t) { return wrapType(t.t.elementType()); })
      .def("get_memory_space", [](const PyMemRefType& t) -> py::object {
        auto s = t.t.memorySpace();
        if (!s) return py::none();
        return py::cast(*s);
      })
      .def("get_layout_map", [](const PyMemRefType& t) {
        return t.t.layout() ? t.t.layout()
                            : AffineMap::multiDimIdentity((unsigned)t.t.rank(), t.t.context());
      });

  py::class_<PyFunctionType, PyType>(m, "function_type", py::module_local())
      .def("param_types", [](const PyFunctionType& t) {
        py::list l;
        for (auto& x : t.t.inputs()) l.append(wrapType(x));
        return l;
      })
      .def("result_types", [](const PyFunctionType& t) {
        py::list l;
        for (auto& x : t.t.results()) l.append(wrapType(x));
        return l;
      });

  py::class_<PyLocation>(m, "location", py::module_local())
      .def("__str__", [](const PyLocation& l) { return l.l.str(); });

  py::class_<PyAttr>(m, "attribute", py::module_local())
      .def("__str__", [](const PyAttr& a) { return a.a.str(); });
  py::class_<PyIntegerAttr, PyAttr>(m, "integer_attr", py::module_local());
  py::class_<PyBoolAttr, PyAttr>(m, "bool_attr", py::module_local());

  py::class_<PyValue>(m, "value", py::module_local())
      .def("get_context", [](const PyValue& v) { return v.v.context(); },
           py::return_value_policy::reference)
      .def("get_defining_op", [](const PyValue& v) { return v.v.definingOp(); },
           py::return_value_policy::reference)
      .def("get_users", [](const PyValue& v) {
        py::list l;
        for (Operation* u : v.v.users()) l.append(py::cast(u, py::return_value_policy::reference));
        return l;
      })
      .def("replace_all_uses_with", [](PyValue& v, const PyValue& n) { v.v.replaceAllUsesWith(n.v); })
      .def("get_type", [](const PyValue& v) { return wrapType(v.v.type()); })
      .def("id", [](const PyValue& v) { return (uint64_t)(uintptr_t)v.v.impl(); })
      .def("__eq__", [](const PyValue& a, const PyValue& b) { return a.v == b.v; })
      .def("__hash__", [](const PyValue& v) { return std::hash<void*>()(v.v.impl()); })
      .def("__repr__", [](const PyValue& v) {
        return "Value(" + std::to_string((uintptr_t)v.v.impl()) + ")";
      })
      .def("__str__", [](const PyValue& v) { return printValueAsOperand(v.v); });
  py::class_<PyOpResult, PyValue>(m, "op_result", py::module_local());
  py::class_<PyBlockArgument, PyValue>(m, "block_argument", py::module_local())
      .def("get_owner", [](const PyBlockArgument& v) { return v.v.ownerBlock(); },
           py::return_value_policy::reference)
      .def("get_arg_number", [](const PyBlockArgument& v) { return v.v.index(); });

  py::class_<PyValueRange>(m, "value_range", py::module_local())
      .def(py::init<>())
      .def(py::init([](const PyValue& v) { return PyValueRange{{v.v}}; }))
      .def(py::init([](const std::vector<PyValue>& vs) { return PyValueRange{unwrapValues(vs)}; }))
      .def("empty", [](const PyValueRange& r) { return r.vals.empty(); })
      .def("size", [](const PyValueRange& r) { return r.vals.size(); })
      .def("__len__", [](const PyValueRange& r) { return r.vals.size(); })
      .def("__getitem__", [](const PyValueRange& r, size_t i) {
        if (i >= r.vals.size()) throw py::index_error("ValueRange index out of range");
        return wrapValue(r.vals[i]);
      })
      .def("__iter__", [](const PyValueRange& r) { return py::iter(wrapValues(r.vals)); })
      .def("to_vector", [](const PyValueRange& r) { return wrapValues(r.vals); })
      .def("__eq__", [](const PyValueRange& a, const PyValueRange& b) { return a.vals == b.vals; })
      .def("__ne__", [](const PyValueRange& a, const PyValueRange& b) { return a.vals != b.vals; })
      .def("__repr__", [](const PyValueRange& r) {
        std::string s = "ValueRange([";
        for (size_t i = 0; i < r.vals.size(); ++i)
          s += (i ? ", " : "") + std::string("Value(") +
               std::to_string((uintptr_t)r.vals[i].impl()) + ")";
        return s + "])";
      })
      .def("__str__", [](const PyValueRange& r) {
        return "ValueRange(size=" + std::to_string(r.vals.size()) + ")";
      });

  py::class_<Region, std::unique_ptr<Region, py::nodelete>>(m, "region", py::module_local())
      .def("get_parent_region", &Region::parentRegion, py::return_value_policy::reference)
      .def("size", &Region::size)
      .def("front", [](Region& r) {
        if (r.empty()) throw py::index_error("region has no blocks");
        return r.front();
      }, py::return_value_policy::reference)
      .def("empty", &Region::empty)
      .def("walk", [](Region& r, const std::function<void(Operation*)>& fn) { r.walk(fn); })
      .def("id", [](Region& r) { return (uint64_t)(uintptr_t)&r; })
      .def("push_back", [](Region& r, Block& b) {
        Context* ctx = r.parent ? r.parent->ctx : nullptr;
        std::unique_ptr<Block> owned = ctx ? ctx->releaseBlock(&b) : nullptr;
        if (!owned) throw InvalidArgument("block already belongs to a region");
        r.pushBack(std::move(owned));
      });

  py::class_<Block, std::unique_ptr<Block, py::nodelete>>(m, "block", py::module_local())
      .def("arg", [](Block& b, int i) {
        if (i < 0 || (unsigned)i >= b.numArguments())
          throw py::index_error("Block argument index out of range");
        return py::cast(PyBlockArgument{{b.argument((unsigned)i)}});
      })
      .def("add_argument", [](Block& b, const PyType& t) { b.addArgument(t.t); })
      .def("get_num_arguments", &Block::numArguments)
      .def("get_argument", [](Block& b, unsigned i) {
        if (i >= b.numArguments()) throw py::index_error("Block argument index out of range");
        return py::cast(PyBlockArgument{{b.argument(i)}});
      })
      .def("dump", [](Block& b) { emitToStderr(printBlock(&b)); })
      .def("move_before", [](Block& self, Block& dst) {
        if (!self.parent || !dst.parent) throw InvalidArgument("blocks must be in regions");
        auto& src = self.parent->blocks;
        auto it = std::find_if(src.begin(), src.end(), [&](auto& p) { return p.get() == &self; });
        auto& dl = dst.parent->blocks;
        auto pos = std::find_if(dl.begin(), dl.end(), [&](auto& p) { return p.get() == &dst; });
        dl.splice(pos, src, it);
        self.parent = dst.parent;
      })
      .def("insert_before", [](Block& self, Block& before) {
        if (!before.parent) throw InvalidArgument("target block is not in a region");
        Region* r = before.parent;
        std::unique_ptr<Block> owned = r->parent->ctx->releaseBlock(&self);
        if (!owned) throw InvalidArgument("block already belongs to a region");
        auto pos = std::find_if(r->blocks.begin(), r->blocks.end(),
                                [&](auto& p) { return p.get() == &before; });
        owned->parent = r;
        r->blocks.insert(pos, std::move(owned));
      })
      .def("get_parent", [](Block& b) { return b.parent; }, py::return_value_policy::reference)
      .def("merge_block_before", [](Block& self, Block& dst) {
        if (self.numArguments()) throw std::runtime_error("This block has arguments, don't merge");
        for (auto& op : self.ops) op->parent = &dst;
        dst.ops.splice(dst.ops.begin(), self.ops);
        if (self.parent) {
          auto& l = self.parent->blocks;
          l.remove_if([&](auto& p) { return p.get() == &self; });
        }
      })
      .def("replace_use_in_block_with", [](Block& self, const PyValue& v, const PyValue& nv) {
        std::vector<Operation*> users = v.v.users();
        for (Operation* u : users) {
          bool inside = false;
          for (Block* b = u->parent; b && !inside; b = b->parentOp() ? b->parentOp()->parent : nullptr)
            inside = b == &self;
          if (!inside) continue;
          for (unsigned i = 0; i < u->numOperands(); ++i)
            if (u->operand(i) == v.v) u->setOperand(i, nv.v);
        }
      })
      .def("__str__", [](Block& b) { return printBlock(&b); })
      .def("has_terminator", [](Block& b) { return b.terminator() != nullptr; })
      .def("has_return", [](Block& b) {
        Operation* t = b.terminator();
        return t && (t->is("func.return") || t->is("scf.yield") || t->is("frisk.end"));
      })
      .def("erase", [](Block& b) {
        if (!b.parent) throw InvalidArgument("block is not in a region");
        b.parent->blocks.remove_if([&](auto& p) { return p.get() == &b; });
      })
      .def("walk", [](Block& b, const std::function<void(Operation*)>& fn) { b.walk(fn); })
      .def("get_operations", [](Block& b) {
        py::list l;
        for (auto& op : b.ops) l.append(py::cast(op.get(), py::return_value_policy::reference));
        return l;
      })
      .def("get_parent_op", [](Block& b) { return b.parentOp(); }, py::return_value_policy::reference)
      .def("id", [](Block& b) { return (uint64_t)(uintptr_t)&b; });

  py::class_<PyInsertPoint>(m, "InsertPoint", py::module_local());
}

// ---- operations ---------------------------------------------------------------
void bindOps(py::module_& m) {
  py::class_<PyOpState>(m, "OpState", py::module_local())
      .def("set_attr", [](PyOpState& s, const std::string& n, const PyAttr& a) {
        requireOp(s)->setAttr(n, a.a);
      })
      .def("get_num_results", [](PyOpState& s) { return requireOp(s)->numResults(); })
      .def("get_result", [](PyOpState& s, unsigned i) {
        Operation* op = requireOp(s);
        if (i >= op->numResults()) throw py::index_error("Op result index out of range");
        return wrapValue(op->result(i));
      })
      .def("get_region", [](PyOpState& s, unsigned i) -> Region& {
        Operation* op = requireOp(s);
        if (i >= op->numRegions()) throw py::index_error("Op region index out of range");
        return op->region(i);
      }, py::return_value_policy::reference)
      .def("get_operation", [](PyOpState& s) { return requireOp(s); },
           py::return_value_policy::reference)
      .def("dump", [](PyOpState& s) { emitToStderr(printOp(requireOp(s))); })
      .def("__str__", [](PyOpState& s) {
        PrintOptions o;
        o.debugInfo = true;
        return printOp(requireOp(s), o);
      })
      .def("append_operand", [](PyOpState& s, const PyValue& v) { requireOp(s)->appendOperand(v.v); })
      .def("verify", [](PyOpState& s) {
        std::string msg = verifyMessage(requireOp(s));
        if (msg.empty()) return true;
        emitToStderr(requireOp(s)->loc.str() + ": error: " + msg);
        return false;
      })
      .def("verify_diagnostic", [](PyOpState& s) -> py::object {
        std::string msg = verifyMessage(requireOp(s));
        if (msg.empty()) return py::none();
        return py::str(msg);
      });

  py::class_<Operation, std::unique_ptr<Operation, py::nodelete>>(m, "operation", py::module_local())
      .def("__str__", [](Operation& o) { return o.name; })
      .def("__repr__", [](Operation& o) { return o.name; })
      .def("get_name", [](Operation& o) { return o.name; })
      .def("get_num_operands", &Operation::numOperands)
      .def("get_operand", [](Operation& o, unsigned i) {
        if (i >= o.numOperands()) throw py::index_error("operand index out of range");
        return wrapValue(o.operand(i));
      })
      .def("set_operand", [](Operation& o, unsigned i, const PyValue& v) { o.setOperand(i, v.v); })
      .def("get_num_results", &Operation::numResults)
      .def("get_result", [](Operation& o, unsigned i) {
        if (i >= o.numResults()) throw py::index_error("result index out of range");
        return wrapValue(o.result(i));
      })
      .def("get_num_regions", &Operation::numRegions)
      .def("get_region", [](Operation& o, unsigned i) -> Region& {
        if (i >= o.numRegions()) throw py::index_error("region index out of range");
        return o.region(i);
      }, py::return_value_policy::reference)
      .def("get_block", [](Operation& o) { return o.parent; }, py::return_value_policy::reference)
      .def("get_parent_op", [](Operation& o) { return o.parentOp(); },
           py::return_value_policy::reference)
      .def("get_str_attr", [](Operation& o, const std::string& n) -> py::object {
        Attribute a = o.attr(n);
        if (!a || a.kind() != AttrKind::String) return py::none();
        return py::str(a->s);
      })
      .def("get_flat_symbol_ref_attr", [](Operation& o, const std::string& n) -> py::object {
        Attribute a = o.attr(n);
        if (!a || a.kind() != AttrKind::String) return py::none();
        return py::str(a->s);
      })
      .def("get_int_attr", [](Operation& o, const std::string& n) -> py::object {
        Attribute a = o.attr(n);
        if (!a || a.kind() != AttrKind::Integer) return py::none();
        return py::int_(a->i);
      })
      .def("get_attr", [](Operation& o, const std::string& n) { return attrToPython(o.attr(n)); })
      .def("get_attr_names", [](Operation& o) {
        std::vector<std::string> names;
        for (auto& a : o.attrs) names.push_back(a.name);
        return names;
      })
      .def("get_operands", [](Operation& o) { return wrapValues(o.operands); })
      .def("get_str", [](Operation& o) { return printOp(&o); })
      .def("is_constant_op", [](Operation& o) { return o.is("arith.constant"); })
      .def("to_constant_op", [](Operation& o) { return opAs<PyConstant>(&o, "arith.constant"); })
      .def("__eq__", [](Operation& a, Operation& b) { return &a == &b; })
      .def("__hash__", [](Operation& a) { return std::hash<void*>()(&a); });

  py::class_<PyModule, PyOpState>(m, "module", py::module_local(), py::dynamic_attr())
      .def("dump", [](PyModule& s, const std::string& log) {
        if (!log.empty()) py::print(log);
        py::print(printOp(requireOp(s)));
      }, py::arg("log") = "")
      .def("__str__", [](PyModule& s) {
        PrintOptions o;
        o.debugInfo = true;
        return printOp(requireOp(s), o);
      })
      .def("push_back", [](PyModule& s, PyOpState& op) {
        Operation* o = requireOp(op);
        if (!o->is("func.func") && !o->is("frisk.kernel"))
          throw InvalidArgument("module.push_back expects a function or kernel");
        if (o->parent == requireOp(s)->body()) return;  // already there
        std::unique_ptr<Operation> owned = o->remove();
        if (!owned) throw InvalidArgument("operation is not owned by this context");
        requireOp(s)->body()->pushBack(std::move(owned));
      })
      .def("has_function", [](PyModule& s, const std::string& n) {
        Operation* o = lookupSymbol(requireOp(s), n);
        return o && o->is("func.func");
      })
      .def("get_function", [](PyModule& s, const std::string& n) {
        return opAs<PyFunc>(lookupSymbol(requireOp(s), n), "func.func");
      })
      .def("get_kernel", [](PyModule& s, const std::string& n) {
        return opAs<PyKernelOp>(lookupSymbol(requireOp(s), n), "frisk.kernel");
      })
      .def("erase_kernel", [](PyModule& s, const std::string& n) {
        Operation* k = lookupSymbol(requireOp(s), n);
        if (!k || !k->is("frisk.kernel")) throw InvalidArgument("no kernel named " + n);
        k->erase();
      })
      .def("get_int_attr", [](PyModule& s, const std::string& n) -> py::object {
        Attribute a = requireOp(s)->attr(n);
        if (!a || a.kind() != AttrKind::Integer) return py::none();
        return py::int_(a->i);
      })
      .def("walk", [](PyModule& s, const std::function<void(Operation*)>& fn) {
        requireOp(s)->walk(fn);
      });

  py::class_<PyConstant, PyOpState>(m, "constant", py::module_local())
      .def("get_splat_float_value", [](PyConstant& s) -> py::object {
        Attribute a = requireOp(s)->attr("value");
        if (a && a.kind() == AttrKind::DenseFloat && a.isSplat()) return py::float_(a->floats[0]);
        return py::none();
      });

  py::class_<PyFunc, PyOpState>(m, "function", py::module_local())
      .def("arg", [](PyFunc& s, unsigned i) {
        Block* b = requireOp(s)->body();
        if (!b || i >= b->numArguments()) throw py::index_error("Function argument index out of range");
        return py::cast(PyBlockArgument{{b->argument(i)}});
      })
      .def("get_num_arguments", [](PyFunc& s) {
        return (unsigned)requireOp(s)->attr("function_type")->type.inputs().size();
      })
      .def("get_callable_region", [](PyFunc& s) -> Region& { return requireOp(s)->region(0); },
           py::return_value_policy::reference)
      .def("get_terminator", [](PyFunc& s) {
        Block* b = requireOp(s)->body();
        return b ? b->terminator() : nullptr;
      }, py::return_value_policy::reference)
      .def("add_entry_block", [](PyFunc& s) { return addFuncEntryBlock(requireOp(s)); },
           py::return_value_policy::reference)
      .def("set_arg_attr", [](PyFunc& s, int argNo, const std::string& name, int val) {
        Operation* op = requireOp(s);
        if (argNo < 0 || (size_t)argNo >= op->attr("function_type")->type.inputs().size())
          throw py::index_error("Function argument index out of range");
        op->setAttr("arg" + std::to_string(argNo) + "." + name,
                    Attribute::integer(op->ctx->integer(32), val));
      })
      .def_property_readonly("type", [](PyFunc& s) {
        return PyFunctionType{{requireOp(s)->attr("function_type")->type}};
      })
      .def("reset_type", [](PyFunc& s, const PyType& t) {
        if (!t.t.isFunction()) throw InvalidArgument("invalid function type");
        requireOp(s)->setAttr("function_type", Attribute::typeAttr(t.t));
      });
}

// ---- builder ------------------------------------------------------------------
void bindBuilder(py::module_& m) {
  py::class_<PyBuilder>(m, "builder")
      .def(py::init<Context*>(), py::keep_alive<1, 2>())
      .def("create_module", [](PyBuilder& b) { return PyModule{{createModule(b.b)}}; })
      .def("set_insertion_point_to_start", [](PyBuilder& b, Block& blk) {
        b.b.setInsertionPointToStart(&blk);
      })
      .def("set_insertion_point_to_end", [](PyBuilder& b, Block& blk) {
        b.b.setInsertionPointToEnd(&blk);
      })
      .def("set_insertion_point_after", [](PyBuilder& b, Operation& op) {
        if (!op.parent) throw InvalidArgument("operation is not in a block");
        b.b.setInsertionPointAfter(&op);
      })
      .def("set_insertion_point_after", [](PyBuilder& b, PyOpState& s) {
        Operation* op = requireOp(s);
        if (!op->parent) throw InvalidArgument("operation is not in a block");
        b.b.setInsertionPointAfter(op);
      })
      .def("get_insertion_block", [](PyBuilder& b) { return b.b.insertionBlock(); },
           py::return_value_policy::reference)
      .def("get_insertion_point", [](PyBuilder& b) { return PyInsertPoint{b.b.saveInsertionPoint()}; })
      .def("restore_insertion_point", [](PyBuilder& b, const PyInsertPoint& ip) {
        b.b.restoreInsertionPoint(ip.ip);
      })
      // Attributes.
      .def("get_bool_attr", [](PyBuilder&, bool v) { return PyBoolAttr{{Attribute::boolean(v)}}; })
      .def("get_int32_attr", [](PyBuilder& b, int32_t v) {
        return PyIntegerAttr{{Attribute::integer(b.b.context()->integer(32), v)}};
      })
      .def("get_str_attr", [](PyBuilder&, const std::string& v) {
        return PyAttr{Attribute::string(v)};
      })
      .def("get_int64_attr", [](PyBuilder& b, int64_t v) {
        return PyIntegerAttr{{Attribute::integer(b.b.context()->integer(64), v)}};
      })
      .def("get_float_attr", [](PyBuilder& b, float v, const std::string& dtype) {
        return PyAttr{Attribute::floating(floatAttrType(b.b.context(), dtype), v)};
      })
      // Extensions for building tensor-form IR directly (the form
      // frisk.normalize_layout_ir produces and layout inference consumes).
      .def("get_gemm_warp_policy_attr", [](PyBuilder&, GemmWarpPolicy p) {
        return PyAttr{Attribute::gemmPolicy(p)};
      })
      .def("get_i64_array_attr", [](PyBuilder&, std::vector<int64_t> v) {
        return PyAttr{Attribute::denseI64(std::move(v))};
      })
      .def("get_dense_splat_attr", [](PyBuilder&, const PyType& tensor, double v) {
        if (!tensor.t.isTensor()) throw InvalidArgument("dense splat needs a tensor type");
        if (tensor.t.elementType().isFloat()) return PyAttr{Attribute::denseFloat(tensor.t, {v})};
        return PyAttr{Attribute::denseInt(tensor.t, {(int64_t)v})};
      })
      .def("create_op", [](PyBuilder& b, const std::string& name, std::vector<PyValue> operands,
                           std::vector<PyType> resultTypes, std::map<std::string, PyAttr> attrs) {
        std::vector<Value> ops;
        for (auto& v : operands) ops.push_back(v.v);
        std::vector<Type> tys;
        for (auto& t : resultTypes) tys.push_back(t.t);
        std::vector<NamedAttr> na;
        for (auto& kv : attrs) na.push_back({kv.first, kv.second.a});
        return PyOpState{b.b.create(name, ops, tys, na)};
      }, py::arg("name"), py::arg("operands"), py::arg("result_types"),
         py::arg("attrs") = std::map<std::string, PyAttr>{})
      // Constants.
      .def("get_int64", [](PyBuilder& b, int64_t v) {
        Type t = b.b.context()->integer(64);
        return wrapValue(createConstant(b.b, Attribute::integer(t, v), t)->result(0));
      })
      .def("get_f16", [](PyBuilder& b, float v) {
        Type t = b.b.context()->floatTy(FloatKind::F16);
        return wrapValue(createConstant(b.b, Attribute::floating(t, v), t)->result(0));
      })
      .def("get_f32", [](PyBuilder& b, float v) {
        Type t = b.b.context()->floatTy(FloatKind::F32);
        return wrapValue(createConstant(b.b, Attribute::floating(t, v), t)->result(0));
      })
      .def("get_f64", [](PyBuilder& b, double v) {
        Type t = b.b.context()->floatTy(FloatKind::F64);
        return wrapValue(createConstant(b.b, Attribute::floating(t, v), t)->result(0));
      })
      .def("get_f16_tensor", [](PyBuilder& b, std::vector<double> v, std::vector<int64_t> shape) {
        Type t = b.b.context()->tensor(shape, b.b.context()->floatTy(FloatKind::F16));
        return wrapValue(createConstant(b.b, Attribute::denseFloat(t, v), t)->result(0));
      })
      .def("get_f32_tensor", [](PyBuilder& b, std::vector<double> v, std::vector<int64_t> shape) {
        Type t = b.b.context()->tensor(shape, b.b.context()->floatTy(FloatKind::F32));
        return wrapValue(createConstant(b.b, Attribute::denseFloat(t, v), t)->result(0));
      })
      .def("get_f64_tensor", [](PyBuilder& b, std::vector<double> v, std::vector<int64_t> shape) {
        Type t = b.b.context()->tensor(shape, b.b.context()->floatTy(FloatKind::F64));
        return wrapValue(createConstant(b.b, Attribute::denseFloat(t, v), t)->result(0));
      })
      .def("get_int64_tensor", [](PyBuilder& b, std::vector<int64_t> v, std::vector<int64_t> shape) {
        Type t = b.b.context()->tensor(shape, b.b.context()->integer(64));
        return wrapValue(createConstant(b.b, Attribute::denseInt(t, v), t)->result(0));
      })
      // Types (get_bool_ty is i8, as in the reference).
      .def("get_bool_ty", [](PyBuilder& b) { return wrapType(b.b.context()->integer(8)); })
      .def("get_int8_ty", [](PyBuilder& b) { return wrapType(b.b.context()->integer(8)); })
      .def("get_int32_ty", [](PyBuilder& b) { return wrapType(b.b.context()->integer(32)); })
      .def("get_int64_ty", [](PyBuilder& b) { return wrapType(b.b.context()->integer(64)); })
      .def("get_index_ty", [](PyBuilder& b) { return wrapType(b.b.context()->index()); })
      .def("get_f64_ty", [](PyBuilder& b) { return wrapType(b.b.context()->floatTy(FloatKind::F64)); })
      .def("get_f16_ty", [](PyBuilder& b) { return wrapType(b.b.context()->floatTy(FloatKind::F16)); })
      .def("get_bf16_ty", [](PyBuilder& b) { return wrapType(b.b.context()->floatTy(FloatKind::BF16)); })
      .def("get_f32_ty", [](PyBuilder& b) { return wrapType(b.b.context()->floatTy(FloatKind::F32)); })
      .def("get_e4m3fn_ty", [](PyBuilder& b) {
        return wrapType(b.b.context()->floatTy(FloatKind::E4M3FN));
      })
      .def("get_e5m2_ty", [](PyBuilder& b) { return wrapType(b.b.context()->floatTy(FloatKind::E5M2)); })
      .def("get_ranked_tensor_ty", [](PyBuilder& b, const PyType& e, std::vector<int64_t> shape) {
        return wrapType(b.b.context()->tensor(shape, e.t));
      })
      .def("get_memref_ty", [](PyBuilder& b, const PyType& e, std::vector<int64_t> shape,
                               AffineMap map, MemorySpace space) {
        return wrapType(b.b.context()->memref(shape, e.t, map, (int64_t)space));
      }, py::arg("elementType"), py::arg("shape"), py::arg("map") = AffineMap(),
         py::arg("space") = MemorySpace::Global)
      .def("get_function_ty", [](PyBuilder& b, std::vector<PyType> ins, std::vector<PyType> outs) {
        return wrapType(b.b.context()->function(unwrapTypes(ins), unwrapTypes(outs)));
      })
      .def("get_kernel_ty", [](PyBuilder& b, std::vector<PyType> ins) {
        return wrapType(b.b.context()->function(unwrapTypes(ins), {}));
      })
      // Locations.
      .def("set_loc", [](PyBuilder& b, const PyLocation& l) { b.b.setLoc(l.l); })
      .def("set_loc", [](PyBuilder& b, const std::string& f, int line, int col) {
        b.b.setLoc(Location{f, line, col});
      })
      .def("get_loc", [](PyBuilder& b) { return PyLocation{currentLoc(b)}; })
      // Structure.
      .def("clone", [](PyBuilder& b, Operation& op) { return b.b.clone(&op); },
           py::return_value_policy::reference)
      .def("get_or_insert_function", [](PyBuilder& b, PyModule& mod, const std::string& name,
                                        const PyType& ft) {
        if (Operation* o = lookupSymbol(requireOp(mod), name)) {
          if (!o->is("func.func")) throw InvalidArgument("symbol '" + name + "' is not a function");
          return PyFunc{{o}};
        }
        return PyFunc{{createFunc(b.b, name, ft.t)}};
      })
      .def("create_block", [](PyBuilder& b) {
        Block* cur = b.b.insertionBlock();
        if (!cur || !cur->parent) throw InvalidArgument("no insertion block");
        Block* nb = cur->parent->emplaceBlock();
        b.b.setInsertionPointToEnd(nb);
        return nb;
      }, py::return_value_policy::reference)
      .def("create_block_with_parent", [](PyBuilder& b, Region& parent, std::vector<PyType> args) {
        Block* nb = parent.emplaceBlock();
        for (auto& t : args) nb->addArgument(t.t);
        b.b.setInsertionPointToEnd(nb);
        return nb;
      }, py::return_value_policy::reference)
      .def("new_block", [](PyBuilder& b) {
        return b.b.context()->adoptBlock(std::make_unique<Block>());
      }, py::return_value_policy::reference)
      .def("ret", [](PyBuilder& b, std::vector<PyValue> vals) {
        return PyOpState{createReturn(b.b, unwrapValues(vals))};
      })
      // Affine helpers.
      .def("get_affine_dim_expr", [](PyBuilder& b, unsigned p) { return getAffineDimExpr(p, b.b.context()); })
      .def("get_affine_symbol_expr", [](PyBuilder& b, unsigned p) {
        return getAffineSymbolExpr(p, b.b.context());
      })
      .def("get_affine_constant_expr", [](PyBuilder& b, int64_t c) {
        return getAffineConstantExpr(c, b.b.context());
      })
      .def("get_empty_affine_map", [](PyBuilder& b) { return AffineMap::get(b.b.context()); })
      .def("get_dim_identity_map", [](PyBuilder& b) { return AffineMap::multiDimIdentity(1, b.b.context()); })
      .def("get_multi_dim_identity_map", [](PyBuilder& b, unsigned r) {
        return AffineMap::multiDimIdentity(r, b.b.context());
      })
      .def("get_symbol_identity_map", [](PyBuilder& b) {
        Context* c = b.b.context();
        return AffineMap::get(0, 1, {getAffineSymbolExpr(0, c)}, c);
      })
      .def("get_single_dim_shift_affine_map", [](PyBuilder& b, int64_t s) {
        Context* c = b.b.context();
        return AffineMap::get(1, 0, {getAffineDimExpr(0, c) + s}, c);
      })
      .def("get_shifted_affine_map", [](PyBuilder&, AffineMap map, int64_t s) {
        std::vector<AffineExpr> r;
        for (auto& e : map.results()) r.push_back(e + s);
        return AffineMap::get(map.numDims(), map.numSymbols(), r, map.context());
      })
      // frisk ops.
      .def("create_gemm_op", [](PyBuilder& b, const PyValue& A, const PyValue& B, const PyValue& C,
                                bool transA, bool transB, bool clear,
                                const std::optional<std::string>& legacy) {
        return PyGemmOp{{createGemm(b.b, A.v, B.v, C.v, transA, transB, clear, legacy)}};
      }, py::arg("A"), py::arg("B"), py::arg("C"), py::arg("transA") = false,
         py::arg("transB") = false, py::arg("clear_accum") = false,
         py::arg("legacy_semantics") = py::none())
      .def("create_kernel_op", [](PyBuilder& b, PyModule& mod, const std::string& name,
                                  const PyType& ty) {
        return PyKernelOp{{createKernel(b.b, requireOp(mod), name, ty.t)}};
      })
      .def("create_parallel_op", [](PyBuilder& b, std::vector<int64_t> grid, int64_t threads) {
        return PyParallelOp{{createParallel(b.b, grid, threads)}};
      })
      .def("create_block_op", [](py::object self, std::vector<int64_t> ranges, py::function fn) {
        PyBuilder& b = self.cast<PyBuilder&>();
        Operation* op = createBlockOp(b.b, ranges, [&](const std::vector<Value>& ivs) {
          runCallback("block op", [&] { fn(self, PyValueRange{ivs}); });
        });
        return PyBlockOp{{op}};
      })
      .def("create_for_op", [](py::object self, int64_t lo, int64_t hi, int64_t step, py::function fn) {
        PyBuilder& b = self.cast<PyBuilder&>();
        Operation* op = createFor(b.b, lo, hi, step, [&](Value iv) {
          runCallback("for op", [&] { fn(self, wrapValue(iv)); });
        });
        return PyForOp{{op}};
      })
      .def("create_alloc_buffer_op", [](PyBuilder& b, std::vector<int64_t> shape,
                                        const std::string& dtype, MemorySpace space, int64_t align) {
        return PyAllocBufferOp{{createAllocBuffer(b.b, shape, dtypeToType(b.b.context(), dtype),
                                                  space, align)}};
      }, py::arg("shape"), py::arg("dtype"), py::arg("space") = MemorySpace::Global,
         py::arg("alignment") = 0)
      .def("create_copy_op", [](PyBuilder& b, const PyValue& src, const PyValue& dst,
                                std::vector<PyValue> srcIdx, std::vector<PyValue> dstIdx,
                                AffineMap srcMap, AffineMap dstMap, std::vector<int64_t> srcExt,
                                std::vector<int64_t> dstExt) {
        return PyCopyOp{{createCopy(b.b, src.v, dst.v, unwrapValues(srcIdx), unwrapValues(dstIdx),
                                    srcMap, dstMap, srcExt, dstExt)}};
      }, py::arg("src"), py::arg("dst"), py::arg("srcIndices"), py::arg("dstIndices"),
         py::arg("srcMap") = AffineMap(), py::arg("dstMap") = AffineMap(),
         py::arg("srcExtents") = std::vector<int64_t>{}, py::arg("dstExtents") = std::vector<int64_t>{})
      .def("create_fill_op", [](PyBuilder& b, const PyValue& memref, float value,
                                const std::string& dtype) {
        Type t = floatAttrType(b.b.context(), dtype);
        return PyFillOp{{createFill(b.b, memref.v, Attribute::floating(t, value))}};
      })
      .def("create_reduce_op", [](PyBuilder& b, const PyValue& src, const PyValue& dst,
                                  const std::string& kind, int64_t dim, bool clear,
                                  const std::optional<std::string>& legacy) {
        return PyReduceOp{{createReduce(b.b, src.v, dst.v, kind, dim, clear, legacy)}};
      }, py::arg("src"), py::arg("dst"), py::arg("kind"), py::arg("dim"), py::arg("clear") = true,
         py::arg("legacy_semantics") = py::none());
}

// ---- CDNA4 layout target ------------------------------------------------------
py::dict instrDict(const MfmaInstr& i) {
  static const char* kinds[] = {"f16", "bf16", "fp8", "i8", "f32"};
  py::dict d;
  d["name"] = i.name;
  d["input"] = kinds[(int)i.input];
  d["m"] = i.m;
  d["n"] = i.n;
  d["k"] = i.k;
  d["in_bits"] = i.inBits;
  d["acc_bits"] = i.accBits;
  return d;
}

void bindLayout(py::module_& m) {
  m.def("mfma_instructions", [] {
    py::list l;
    for (auto& i : cdna4MfmaTable()) l.append(instrDict(i));
    return l;
  });

  py::class_<MmaGeometry>(m, "MmaGeometry")
      .def_readonly("m", &MmaGeometry::m)
      .def_readonly("n", &MmaGeometry::n)
      .def_readonly("k", &MmaGeometry::k)
      .def_readonly("threads", &MmaGeometry::threads)
      .def_readonly("gM", &MmaGeometry::gM)
      .def_readonly("gN", &MmaGeometry::gN)
      .def_readonly("mRepeat", &MmaGeometry::mRepeat)
      .def_readonly("nRepeat", &MmaGeometry::nRepeat)
      .def_readonly("kRepeat", &MmaGeometry::kRepeat)
      .def_property_readonly("atom", [](const MmaGeometry& g) { return instrDict(g.atom); })
      .def_property_readonly("waves", &MmaGeometry::waves)
      .def("registers", [](const MmaGeometry& g, const std::string& op) {
        if (op == "A") return g.aRegs();
        if (op == "B") return g.bRegs();
        if (op == "C") return g.cRegs();
        throw InvalidArgument("operand must be 'A', 'B' or 'C'");
      })
      .def("coordinate", [](const MmaGeometry& g, const std::string& op, int64_t reg, int64_t lane,
                            int64_t wave) {
        if (op != "A" && op != "B" && op != "C") throw InvalidArgument("operand must be 'A', 'B' or 'C'");
        const int64_t regs = op == "A" ? g.aRegs() : op == "B" ? g.bRegs() : g.cRegs();
        if (reg < 0 || reg >= regs || lane < 0 || lane >= 64 || wave < 0 || wave >= g.waves())
          throw py::index_error("fragment coordinate out of range");
        auto rc = cdna4FragmentCoordinate(g, op[0], reg, lane, wave);
        return py::make_tuple(rc[0], rc[1]);
      })
      .def("gf2", [](const MmaGeometry& g, const std::string& op) -> py::object {
        if (op != "A" && op != "B" && op != "C") throw InvalidArgument("operand must be 'A', 'B' or 'C'");
        auto map = cdna4FragmentGf2(g, op[0]);
        if (!map) return py::none();
        py::dict d;
        d["in_bits"] = map->inBits;
        d["out_bits"] = map->outBits;
        d["cols"] = map->cols;
        d["rank"] = map->rank();
        return d;
      })
      .def("__repr__", [](const MmaGeometry& g) {
        return "MmaGeometry(" + std::to_string(g.m) + "x" + std::to_string(g.n) + "x" +
               std::to_string(g.k) + ", threads=" + std::to_string(g.threads) + ", grid=" +
               std::to_string(g.gM) + "x" + std::to_string(g.gN) + ", atom=" + g.atom.name + ")";
      });

  m.def("mma_geometry", [](int64_t mm, int64_t n, int64_t k, const PyType& in, const PyType& acc,
                           int64_t threads, GemmWarpPolicy policy) -> py::object {
    auto g = cdna4MmaGeometry(mm, n, k, in.t, acc.t, threads, policy);
    if (!g) return py::none();
    return py::cast(*g);
  }, py::arg("m"), py::arg("n"), py::arg("k"), py::arg("in_type"), py::arg("acc_type"),
     py::arg("threads") = 256, py::arg("policy") = GemmWarpPolicy::Square);

  py::class_<SwizzleProposal>(m, "SwizzleProposal")
      .def_readonly("row_bytes", &SwizzleProposal::rowBytes)
      .def_readonly("read_conflict", &SwizzleProposal::readConflict)
      .def_readonly("formula", &SwizzleProposal::formula)
      .def_property_readonly("terms", [](const SwizzleProposal& p) {
        py::list l;
        for (auto& t : p.terms) l.append(py::make_tuple(t.shift, t.mask, t.lshift));
        return l;
      })
      .def("chunk", &SwizzleProposal::chunk, py::arg("row"), py::arg("chunk"))
      .def("offset", &SwizzleProposal::offset, py::arg("row"), py::arg("byte"))
      .def("__repr__", [](const SwizzleProposal& p) {
        return "SwizzleProposal(row_bytes=" + std::to_string(p.rowBytes) + ", " + p.formula + ")";
      });
  m.def("lds_swizzle", &proposeLdsSwizzle, py::arg("row_bytes"), py::arg("atom_m") = 32);
  m.def("lds_read_b128_conflict", &ldsReadB128ConflictFactor, py::arg("addresses"));
  m.def("sm90_swizzle", &sm90StyleSwizzle, py::arg("offset"), py::arg("swizzle_bytes"));
}

// ---- ir.frisk -----------------------------------------------------------------
void bindFrisk(py::module_& m) {
  m.def("load_dialects", [](Context& c) { c.dialectsLoaded = true; });

  py::class_<PyGemmOp, PyOpState>(m, "GemmOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyGemmOp>(&o, "frisk.gemm"); })
      .def("get_matrix_A", [](PyGemmOp& s) { return wrapValue(requireOp(s)->operand(0)); })
      .def("get_matrix_B", [](PyGemmOp& s) { return wrapValue(requireOp(s)->operand(1)); })
      .def("get_matrix_C", [](PyGemmOp& s) { return wrapValue(requireOp(s)->operand(2)); })
      .def("get_all_matrix", [](PyGemmOp& s) { return PyValueRange{requireOp(s)->operands}; });

  py::class_<PyKernelOp, PyOpState>(m, "KernelOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyKernelOp>(&o, "frisk.kernel"); })
      .def("arg", [](PyKernelOp& s, unsigned i) {
        Block* b = requireOp(s)->body();
        if (!b || i >= b->numArguments()) throw py::index_error("Kernel argument index out of range");
        return py::cast(PyBlockArgument{{b->argument(i)}});
      })
      .def("get_num_arguments", [](PyKernelOp& s) {
        Block* b = requireOp(s)->body();
        return b ? b->numArguments() : 0u;
      })
      .def("add_entry_block", [](PyKernelOp& s) { return addKernelEntryBlock(requireOp(s)); },
           py::return_value_policy::reference)
      .def_property_readonly("type", [](PyKernelOp& s) {
        return PyFunctionType{{requireOp(s)->attr("function_type")->type}};
      });

  py::class_<PyParallelOp, PyOpState>(m, "ParallelOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyParallelOp>(&o, "frisk.parallel"); })
      .def("get_ivs", [](PyParallelOp& s) {
        py::list l;
        if (Block* b = requireOp(s)->body())
          for (unsigned i = 0; i < b->numArguments(); ++i) l.append(PyBlockArgument{{b->argument(i)}});
        return l;
      })
      .def("get_grid", [](PyParallelOp& s) { return i64Array(requireOp(s), "ranges"); })
      .def("get_thread_num", [](PyParallelOp& s) { return requireOp(s)->intAttr("threads"); })
      .def("get_grid_dim", [](PyParallelOp& s) { return i64Array(requireOp(s), "ranges").size(); })
      .def("add_entry_block", [](PyParallelOp& s) { return addParallelEntryBlock(requireOp(s)); },
           py::return_value_policy::reference);

  py::class_<PyBlockOp, PyOpState>(m, "BlockOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyBlockOp>(&o, "frisk.block"); })
      .def("get_ivs", [](PyBlockOp& s) {
        py::list l;
        if (Block* b = requireOp(s)->body())
          for (unsigned i = 0; i < b->numArguments(); ++i) l.append(PyBlockArgument{{b->argument(i)}});
        return l;
      })
      .def("get_block_ranges", [](PyBlockOp& s) { return i64Array(requireOp(s), "ranges"); })
      .def("get_iteration_num", [](PyBlockOp& s) {
        auto r = i64Array(requireOp(s), "ranges");
        return std::accumulate(r.begin(), r.end(), (int64_t)1, std::multiplies<int64_t>());
      })
      .def("get_block_dim", [](PyBlockOp& s) { return i64Array(requireOp(s), "ranges").size(); });

  py::class_<PyForOp, PyOpState>(m, "ForOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyForOp>(&o, "frisk.for"); })
      .def("get_induction_var", [](PyForOp& s) {
        return py::cast(PyBlockArgument{{requireOp(s)->body()->argument(0)}});
      })
      .def("get_lower_bound", [](PyForOp& s) { return requireOp(s)->intAttr("lower"); })
      .def("get_upper_bound", [](PyForOp& s) { return requireOp(s)->intAttr("upper"); })
      .def("get_step", [](PyForOp& s) { return requireOp(s)->intAttr("step"); });

  auto space = [](PyAllocBufferOp& s) { return (MemorySpace)requireOp(s)->intAttr("memorySpace"); };
  py::class_<PyAllocBufferOp, PyOpState>(m, "AllocBufferOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyAllocBufferOp>(&o, "frisk.alloc_buffer"); })
      .def("get_alignment", [](PyAllocBufferOp& s) { return requireOp(s)->intAttr("alignment"); })
      .def("get_memroy_space", space)
      .def("get_memory_space", space)
      .def("get_result", [](PyAllocBufferOp& s) { return wrapValue(requireOp(s)->result(0)); })
      .def("get_memref_ty", [](PyAllocBufferOp& s) { return wrapType(requireOp(s)->result(0).type()); });

  py::class_<PyCopyOp, PyOpState>(m, "CopyOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyCopyOp>(&o, "frisk.copy"); })
      .def("get_src_affine_map", [](PyCopyOp& s) { return copyParts(requireOp(s)).srcMap; })
      .def("get_dst_affine_map", [](PyCopyOp& s) { return copyParts(requireOp(s)).dstMap; })
      .def("get_src_memref", [](PyCopyOp& s) { return wrapValue(copyParts(requireOp(s)).src); })
      .def("get_dst_memref", [](PyCopyOp& s) { return wrapValue(copyParts(requireOp(s)).dst); })
      .def("get_src_memref_ty", [](PyCopyOp& s) { return wrapType(copyParts(requireOp(s)).src.type()); })
      .def("get_dst_memref_ty", [](PyCopyOp& s) { return wrapType(copyParts(requireOp(s)).dst.type()); })
      .def("get_src_indices", [](PyCopyOp& s) { return PyValueRange{copyParts(requireOp(s)).srcIdx}; })
      .def("get_dst_indices", [](PyCopyOp& s) { return PyValueRange{copyParts(requireOp(s)).dstIdx}; })
      .def("get_src_extents", [](PyCopyOp& s) { return copyParts(requireOp(s)).srcExtents; })
      .def("get_dst_extents", [](PyCopyOp& s) { return copyParts(requireOp(s)).dstExtents; });

  py::class_<PyFillOp, PyOpState>(m, "FillOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyFillOp>(&o, "frisk.fill"); })
      .def("get_memref", [](PyFillOp& s) { return wrapValue(requireOp(s)->operand(0)); });

  py::class_<PyReduceOp, PyOpState>(m, "ReduceOp", py::module_local())
      .def_static("from_operation", [](Operation& o) { return opAs<PyReduceOp>(&o, "frisk.reduce"); })
      .def("get_src_memref", [](PyReduceOp& s) { return wrapValue(requireOp(s)->operand(0)); })
      .def("get_dst_memref", [](PyReduceOp& s) { return wrapValue(requireOp(s)->operand(1)); })
      .def("get_reduce_dim", [](PyReduceOp& s) { return requireOp(s)->intAttr("dim"); });

  // Pass: legacy tile ops -> tensor-form ops (frisk-normalize-layout-ir).
  // `target` (optional) is stored as the module's frisk.target first.
  m.def("normalize_layout_ir", [](PyModule& mod, std::optional<std::string> target) {
    if (target) requireOp(mod)->setAttr("frisk.target", Attribute::string(*target));
    std::string err = normalizeLegacyFragments(requireOp(mod));
    if (!err.empty()) throw InvalidArgument(err);
  }, py::arg("module"), py::arg("target") = py::none());

  // Pass: frisk-infer-layouts for gfx950 (layout inference, cost model,
  // materialization).  Returns the solver report as a dict.
  m.def("infer_layouts", [](PyModule& mod, std::optional<std::string> target, int64_t exactLimit,
                            int64_t beamWidth, int64_t maxExpanded, bool analysisOnly,
                            std::optional<std::string> costProfile) {
    Operation* op = requireOp(mod);
    if (target) op->setAttr("frisk.target", Attribute::string(*target));
    InferOptions o;
    o.exactCombinationLimit = exactLimit;
    o.beamWidth = beamWidth;
    o.maxExpandedStates = maxExpanded;
    o.analysisOnly = analysisOnly;
    if (costProfile) o.profile = CostProfile::fromJson(*costProfile);
    InferReport r = inferLayouts(op, o);
    if (r.status == "failed") throw InvalidArgument(r.failure.empty() ? "layout-inference failed" : r.failure);
    py::dict d;
    d["status"] = r.status;
    d["method"] = r.method;
    d["cost_model"] = r.costModelId;
    d["cost"] = r.cost;
    d["variables"] = r.variables;
    d["combinations"] = r.combinations;
    d["expanded"] = r.expanded;
    d["conversions_inserted"] = r.conversionsInserted;
    d["features"] = r.features;
    d["assignments"] = r.assignments;
    d["conversions"] = r.conversions;
    d["graph"] = r.graph;
    return d;
  }, py::arg("module"), py::arg("target") = py::none(), py::arg("exact_combination_limit") = 256,
     py::arg("beam_width") = 32, py::arg("max_expanded_states") = 65536,
     py::arg("analysis_only") = false, py::arg("cost_profile") = py::none());
  // Pass: frisk-export-execution -> the execution packet as JSON text.
  m.def("print_module", [](PyModule& mod, bool debugInfo) {
    PrintOptions o;
    o.debugInfo = debugInfo;
    return printOp(requireOp(mod), o);
  }, py::arg("module"), py::arg("debug_info") = false);
  m.def("parse_module", [](const std::string& text, Context& ctx) {
    return PyModule{{parseModule(&ctx, text)}};
  }, py::arg("text"), py::arg("context"));
  m.def("export_execution", [](PyModule& mod) {
    std::string err;
    std::string out = exportExecution(requireOp(mod), &err);
    if (out.empty()) throw InvalidArgument(err);
    return out;
  }, py::arg("module"));
  m.def("gemm_launch_plan", [](int64_t mm, int64_t n, int64_t k, const PyType& in, const PyType& out,
                               bool transA, bool transB, int64_t cus, bool workspace,
                               bool matrixCores) {
    const GemmLaunchContract c =
        cdna4GemmLaunch(mm, n, k, in.t, out.t, transA, transB, cus, workspace, matrixCores);
    py::dict d;
    d["kernel"] = c.kernel;
    d["tile"] = std::vector<int64_t>{c.tileM, c.tileN};
    d["wave_grid"] = std::vector<int64_t>{c.waveM, c.waveN};
    d["stage_bytes"] = c.stageBytes;
    d["slices"] = c.slices;
    d["kb_slice"] = c.kbSlice;
    d["slice_sum"] = c.sliceSum;
    d["workspace_bytes"] = c.workspaceBytes;
    d["lds_swizzle_a"] = c.swizzleA;
    d["lds_swizzle_b"] = c.swizzleB;
    d["contract"] = c.str();
    return d;
  }, py::arg("m"), py::arg("n"), py::arg("k"), py::arg("in_type"), py::arg("out_type"),
     py::arg("trans_a") = false, py::arg("trans_b") = false, py::arg("cus") = 256,
     py::arg("workspace") = true, py::arg("matrix_cores") = true);
  m.def("attention_launch_plan", [](int64_t batchHeads, int64_t seqQ, int64_t headDim, bool causal,
                                    int64_t cus) {
    py::dict d;
    d["waves"] = cdna4AttentionWaves(batchHeads, seqQ, headDim, causal, cus);
    return d;
  }, py::arg("batch_heads"), py::arg("seq_q"), py::arg("head_dim"), py::arg("causal") = false,
     py::arg("cus") = 256);
  m.def("cost_profile_defaults", []() {
    CostProfile p = CostProfile::defaults();
    py::dict d;
    d["id"] = p.id;
    d["weights"] = p.weights;
    d["simd_share"] = p.simdShare;
    d["per_wave"] = CostProfile::perWaveFeatures();
    return d;
  });
  m.def("mma_bindings", [](int64_t mm, int64_t n, int64_t k, const PyType& in, const PyType& acc,
                           int64_t threads, GemmWarpPolicy policy) {
    py::list out;
    for (const MmaBinding& b : cdna4MmaBindings(mm, n, k, in.t, acc.t, threads, policy)) {
      py::dict d;
      d["atom"] = std::string(b.hw.atom.name);
      d["wave_grid"] = std::vector<int64_t>{b.hw.gM, b.hw.gN};
      d["swapped"] = b.swapped;
      d["contract"] = b.str();
      d["a"] = b.operand('A').str();
      d["b"] = b.operand('B').str();
      d["c"] = b.operand('C').str();
      d["mfma_per_wave"] = b.mfmaPerWave();
      out.append(d);
    }
    return out;
  }, py::arg("m"), py::arg("n"), py::arg("k"), py::arg("in_type"), py::arg("acc_type"),
     py::arg("threads") = 256, py::arg("policy") = GemmWarpPolicy::Auto);

  bindLayout(m);
}

}  // namespace

PYBIND11_MODULE(frisk_ffi, m) {
  m.doc() = "Frisk tile IR builder for MI355X (gfx950)";
  py::module_ ir = m.def_submodule("ir", "tile IR builder");
  bindAffine(ir);
  bindCore(ir);
  bindOps(ir);
  bindBuilder(ir);
  py::module_ frisk = ir.def_submodule("frisk", "frisk dialect ops");
  bindFrisk(frisk);
}
