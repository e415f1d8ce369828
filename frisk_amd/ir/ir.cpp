// Core of the host tile IR: affine expressions/maps, types, attributes,
// values, operations, blocks, regions, the uniquing Context and the Builder.
#include "ir.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <sstream>

namespace fir {

// ============================================================================
// Affine expressions
// ============================================================================
namespace {

int64_t floorDivInt(int64_t a, int64_t b) {
  int64_t q = a / b, r = a % b;
  return (r != 0 && ((r < 0) != (b < 0))) ? q - 1 : q;
}
int64_t ceilDivInt(int64_t a, int64_t b) { return -floorDivInt(-a, b); }
int64_t modInt(int64_t a, int64_t b) { return a - floorDivInt(a, b) * b; }

const AffineExprStorage* constOf(AffineExpr e) {
  return (e && e.kind() == AffineKind::Constant) ? e.impl() : nullptr;
}

Context* ctxOf(AffineExpr a, AffineExpr b) {
  if (!a || !b) throw InvalidArgument("null affine expression");
  if (a.context() != b.context()) throw InvalidArgument("affine expressions from different contexts");
  return a.context();
}

AffineExpr make(Context* c, AffineKind k, AffineExpr l, AffineExpr r) {
  return AffineExpr(c->uniqueExpr(k, 0, l.impl(), r.impl()));
}

AffineExpr simplifyAdd(AffineExpr a, AffineExpr b) {
  Context* c = ctxOf(a, b);
  auto ca = constOf(a), cb = constOf(b);
  if (ca && cb) return getAffineConstantExpr(ca->value + cb->value, c);
  if (ca) std::swap(a, b), std::swap(ca, cb);  // constant to the right
  if (cb && cb->value == 0) return a;
  // (x + c1) + c2 -> x + (c1 + c2)
  if (cb && a.kind() == AffineKind::Add) {
    if (auto c1 = constOf(a.rhs())) return a.lhs() + (c1->value + cb->value);
  }
  // x + (y + c) -> (x + y) + c keeps constants outermost on the right.
  if (b.kind() == AffineKind::Add && constOf(b.rhs())) return (a + b.lhs()) + b.rhs();
  return make(c, AffineKind::Add, a, b);
}

AffineExpr simplifyMul(AffineExpr a, AffineExpr b) {
  Context* c = ctxOf(a, b);
  auto ca = constOf(a), cb = constOf(b);
  if (ca && cb) return getAffineConstantExpr(ca->value * cb->value, c);
  if (ca) std::swap(a, b), std::swap(ca, cb);
  if (cb && cb->value == 1) return a;
  if (cb && cb->value == 0) return b;
  // (x * c1) * c2 -> x * (c1 * c2)
  if (cb && a.kind() == AffineKind::Mul) {
    if (auto c1 = constOf(a.rhs())) return a.lhs() * (c1->value * cb->value);
  }
  return make(c, AffineKind::Mul, a, b);
}

AffineExpr simplifyDivMod(AffineKind k, AffineExpr a, AffineExpr b) {
  Context* c = ctxOf(a, b);
  auto ca = constOf(a), cb = constOf(b);
  if (cb && cb->value == 0) throw InvalidArgument("affine division by zero");
  if (ca && cb) {
    int64_t x = ca->value, y = cb->value;
    int64_t v = k == AffineKind::Mod ? modInt(x, y)
                : k == AffineKind::FloorDiv ? floorDivInt(x, y) : ceilDivInt(x, y);
    return getAffineConstantExpr(v, c);
  }
  if (cb && cb->value == 1) return k == AffineKind::Mod ? getAffineConstantExpr(0, c) : a;
  if (cb && cb->value > 0 && k == AffineKind::Mod && a.isMultipleOf(cb->value))
    return getAffineConstantExpr(0, c);
  // (x * c1) floordiv c2 with c1 % c2 == 0 -> x * (c1 / c2)
  if (cb && cb->value > 0 && k != AffineKind::Mod && a.kind() == AffineKind::Mul) {
    if (auto c1 = constOf(a.rhs()); c1 && c1->value % cb->value == 0)
      return a.lhs() * (c1->value / cb->value);
  }
  return make(c, k, a, b);
}

}  // namespace

bool AffineExpr::operator==(int64_t v) const {
  return s_ && s_->kind == AffineKind::Constant && s_->value == v;
}
Context* AffineExpr::context() const { return s_ ? s_->ctx : nullptr; }
AffineKind AffineExpr::kind() const {
  if (!s_) throw InvalidArgument("null affine expression");
  return s_->kind;
}

AffineExpr getAffineDimExpr(unsigned pos, Context* ctx) {
  return AffineExpr(ctx->uniqueExpr(AffineKind::DimId, pos, nullptr, nullptr));
}
AffineExpr getAffineSymbolExpr(unsigned pos, Context* ctx) {
  return AffineExpr(ctx->uniqueExpr(AffineKind::SymbolId, pos, nullptr, nullptr));
}
AffineExpr getAffineConstantExpr(int64_t v, Context* ctx) {
  return AffineExpr(ctx->uniqueExpr(AffineKind::Constant, v, nullptr, nullptr));
}
AffineExpr getAffineBinaryOpExpr(AffineKind kind, AffineExpr lhs, AffineExpr rhs) {
  switch (kind) {
    case AffineKind::Add: return lhs + rhs;
    case AffineKind::Mul: return lhs * rhs;
    case AffineKind::Mod: return lhs % rhs;
    case AffineKind::FloorDiv: return floorDiv(lhs, rhs);
    case AffineKind::CeilDiv: return ceilDiv(lhs, rhs);
    default: throw InvalidArgument("not a binary affine expression kind");
  }
}

AffineExpr operator+(AffineExpr a, AffineExpr b) { return simplifyAdd(a, b); }
AffineExpr operator+(AffineExpr a, int64_t b) { return a + getAffineConstantExpr(b, a.context()); }
AffineExpr operator*(AffineExpr a, AffineExpr b) { return simplifyMul(a, b); }
AffineExpr operator*(AffineExpr a, int64_t b) { return a * getAffineConstantExpr(b, a.context()); }
AffineExpr operator-(AffineExpr a) { return a * int64_t(-1); }
AffineExpr operator-(AffineExpr a, AffineExpr b) { return a + (-b); }
AffineExpr operator-(AffineExpr a, int64_t b) { return a + (-b); }
AffineExpr operator%(AffineExpr a, AffineExpr b) { return simplifyDivMod(AffineKind::Mod, a, b); }
AffineExpr operator%(AffineExpr a, uint64_t b) {
  return a % getAffineConstantExpr((int64_t)b, a.context());
}
AffineExpr floorDiv(AffineExpr a, AffineExpr b) { return simplifyDivMod(AffineKind::FloorDiv, a, b); }
AffineExpr floorDiv(AffineExpr a, uint64_t b) {
  return floorDiv(a, getAffineConstantExpr((int64_t)b, a.context()));
}
AffineExpr ceilDiv(AffineExpr a, AffineExpr b) { return simplifyDivMod(AffineKind::CeilDiv, a, b); }
AffineExpr ceilDiv(AffineExpr a, uint64_t b) {
  return ceilDiv(a, getAffineConstantExpr((int64_t)b, a.context()));
}

bool AffineExpr::isSymbolicOrConstant() const {
  switch (kind()) {
    case AffineKind::Constant: case AffineKind::SymbolId: return true;
    case AffineKind::DimId: return false;
    default: return lhs().isSymbolicOrConstant() && rhs().isSymbolicOrConstant();
  }
}

bool AffineExpr::isPureAffine() const {
  switch (kind()) {
    case AffineKind::Constant: case AffineKind::SymbolId: case AffineKind::DimId: return true;
    case AffineKind::Add: return lhs().isPureAffine() && rhs().isPureAffine();
    case AffineKind::Mul:
      return lhs().isPureAffine() && rhs().isPureAffine() &&
             (lhs().isSymbolicOrConstant() || rhs().isSymbolicOrConstant());
    default: return lhs().isPureAffine() && rhs().kind() == AffineKind::Constant;
  }
}

int64_t AffineExpr::largestKnownDivisor() const {
  switch (kind()) {
    case AffineKind::Constant: return std::llabs(value());
    case AffineKind::SymbolId: case AffineKind::DimId: return 1;
    case AffineKind::Mul: return lhs().largestKnownDivisor() * rhs().largestKnownDivisor();
    case AffineKind::Add: case AffineKind::Mod:
      return std::gcd(lhs().largestKnownDivisor(), rhs().largestKnownDivisor());
    default: {
      auto c = constOf(rhs());
      int64_t d = lhs().largestKnownDivisor();
      if (c && c->value != 0 && d % c->value == 0) return std::llabs(d / c->value);
      return 1;
    }
  }
}

bool AffineExpr::isMultipleOf(int64_t f) const {
  if (f == 0) return false;
  if (kind() == AffineKind::Constant) return value() % f == 0;
  return largestKnownDivisor() % f == 0;
}

bool AffineExpr::isFunctionOfDim(unsigned pos) const {
  if (kind() == AffineKind::DimId) return position() == pos;
  if (isBinary()) return lhs().isFunctionOfDim(pos) || rhs().isFunctionOfDim(pos);
  return false;
}
bool AffineExpr::isFunctionOfSymbol(unsigned pos) const {
  if (kind() == AffineKind::SymbolId) return position() == pos;
  if (isBinary()) return lhs().isFunctionOfSymbol(pos) || rhs().isFunctionOfSymbol(pos);
  return false;
}

AffineExpr AffineExpr::replaceDimsAndSymbols(const std::vector<AffineExpr>& dims,
                                             const std::vector<AffineExpr>& syms) const {
  switch (kind()) {
    case AffineKind::Constant: return *this;
    case AffineKind::DimId: return position() < dims.size() ? dims[position()] : *this;
    case AffineKind::SymbolId: return position() < syms.size() ? syms[position()] : *this;
    default:
      return getAffineBinaryOpExpr(kind(), lhs().replaceDimsAndSymbols(dims, syms),
                                   rhs().replaceDimsAndSymbols(dims, syms));
  }
}

AffineExpr AffineExpr::replace(const std::map<const AffineExprStorage*, AffineExpr>& m) const {
  auto it = m.find(s_);
  if (it != m.end()) return it->second;
  if (!isBinary()) return *this;
  return getAffineBinaryOpExpr(kind(), lhs().replace(m), rhs().replace(m));
}

AffineExpr AffineExpr::shiftDims(unsigned numDims, unsigned shift, unsigned offset) const {
  std::vector<AffineExpr> dims;
  for (unsigned i = 0; i < numDims; ++i)
    dims.push_back(getAffineDimExpr(i < offset ? i : i + shift, context()));
  return replaceDimsAndSymbols(dims, {});
}
AffineExpr AffineExpr::shiftSymbols(unsigned numSyms, unsigned shift, unsigned offset) const {
  std::vector<AffineExpr> syms;
  for (unsigned i = 0; i < numSyms; ++i)
    syms.push_back(getAffineSymbolExpr(i < offset ? i : i + shift, context()));
  return replaceDimsAndSymbols({}, syms);
}

int64_t AffineExpr::eval(const std::vector<int64_t>& dims, const std::vector<int64_t>& syms) const {
  switch (kind()) {
    case AffineKind::Constant: return value();
    case AffineKind::DimId:
      if (position() >= dims.size()) throw InvalidArgument("affine dim out of range");
      return dims[position()];
    case AffineKind::SymbolId:
      if (position() >= syms.size()) throw InvalidArgument("affine symbol out of range");
      return syms[position()];
    default: {
      int64_t a = lhs().eval(dims, syms), b = rhs().eval(dims, syms);
      switch (kind()) {
        case AffineKind::Add: return a + b;
        case AffineKind::Mul: return a * b;
        default:
          if (b == 0) throw InvalidArgument("affine division by zero");
          if (kind() == AffineKind::Mod) return modInt(a, b);
          if (kind() == AffineKind::FloorDiv) return floorDivInt(a, b);
          return ceilDivInt(a, b);
      }
    }
  }
}

namespace {
// Print with MLIR's two binding strengths: an operand of *, mod and div is
// printed "strong" (binary expressions parenthesised), + operands "weak".
void printExpr(std::ostream& os, AffineExpr e, bool strong) {
  switch (e.kind()) {
    case AffineKind::Constant: os << e.value(); return;
    case AffineKind::DimId: os << 'd' << e.position(); return;
    case AffineKind::SymbolId: os << 's' << e.position(); return;
    default: break;
  }
  if (strong) os << '(';
  if (e.kind() == AffineKind::Add) {
    AffineExpr r = e.rhs();
    auto neg_const = constOf(r);
    if (r.kind() == AffineKind::Mul && constOf(r.rhs()) && constOf(r.rhs())->value < 0) {
      int64_t v = constOf(r.rhs())->value;
      printExpr(os, e.lhs(), false);
      os << " - ";
      printExpr(os, r.lhs(), v != -1 || r.lhs().kind() == AffineKind::Add);
      if (v != -1) os << " * " << -v;
    } else if (neg_const && neg_const->value < 0) {
      printExpr(os, e.lhs(), false);
      os << " - " << -neg_const->value;
    } else {
      printExpr(os, e.lhs(), false);
      os << " + ";
      printExpr(os, r, false);
    }
  } else {
    const char* op = e.kind() == AffineKind::Mul ? " * "
                     : e.kind() == AffineKind::Mod ? " mod "
                     : e.kind() == AffineKind::FloorDiv ? " floordiv " : " ceildiv ";
    printExpr(os, e.lhs(), true);
    os << op;
    printExpr(os, e.rhs(), true);
  }
  if (strong) os << ')';
}
}  // namespace

std::string AffineExpr::str() const {
  if (!s_) return "<<NULL AFFINE EXPR>>";
  std::ostringstream os;
  printExpr(os, *this, false);
  return os.str();
}

// ============================================================================
// Affine maps
// ============================================================================
AffineMap AffineMap::get(Context* ctx) { return AffineMap(ctx->uniqueMap(0, 0, {})); }
AffineMap AffineMap::get(unsigned dims, unsigned syms, Context* ctx) {
  return AffineMap(ctx->uniqueMap(dims, syms, {}));
}
AffineMap AffineMap::get(unsigned dims, unsigned syms, AffineExpr result) {
  return AffineMap(result.context()->uniqueMap(dims, syms, {result}));
}
AffineMap AffineMap::get(unsigned dims, unsigned syms, const std::vector<AffineExpr>& results,
                         Context* ctx) {
  for (auto& r : results) {
    if (!r) throw InvalidArgument("null affine expression in map");
    if (r.context() != ctx) throw InvalidArgument("affine expression from another context");
  }
  return AffineMap(ctx->uniqueMap(dims, syms, results));
}
AffineMap AffineMap::constantMap(int64_t v, Context* ctx) {
  return get(0, 0, {getAffineConstantExpr(v, ctx)}, ctx);
}
AffineMap AffineMap::multiDimIdentity(unsigned dims, Context* ctx) {
  std::vector<AffineExpr> r;
  for (unsigned i = 0; i < dims; ++i) r.push_back(getAffineDimExpr(i, ctx));
  return get(dims, 0, r, ctx);
}
AffineMap AffineMap::minorIdentity(unsigned dims, unsigned results, Context* ctx) {
  if (results > dims) throw InvalidArgument("minor identity needs results <= dims");
  std::vector<AffineExpr> r;
  for (unsigned i = dims - results; i < dims; ++i) r.push_back(getAffineDimExpr(i, ctx));
  return get(dims, 0, r, ctx);
}
AffineMap AffineMap::permutation(const std::vector<unsigned>& perm, Context* ctx) {
  std::vector<bool> seen(perm.size(), false);
  std::vector<AffineExpr> r;
  for (unsigned p : perm) {
    if (p >= perm.size() || seen[p]) throw InvalidArgument("not a permutation");
    seen[p] = true;
    r.push_back(getAffineDimExpr(p, ctx));
  }
  return get((unsigned)perm.size(), 0, r, ctx);
}

const std::vector<AffineExpr>& AffineMap::results() const {
  static const std::vector<AffineExpr> empty;
  return s_ ? s_->results : empty;
}
AffineExpr AffineMap::result(unsigned i) const {
  if (i >= numResults()) throw std::out_of_range("affine map result index out of range");
  return s_->results[i];
}
bool AffineMap::isIdentity() const {
  if (!s_ || numDims() != numResults()) return false;
  for (unsigned i = 0; i < numResults(); ++i)
    if (result(i).kind() != AffineKind::DimId || result(i).position() != i) return false;
  return true;
}
bool AffineMap::isSymbolIdentity() const {
  if (!s_ || numSymbols() != numResults()) return false;
  for (unsigned i = 0; i < numResults(); ++i)
    if (result(i).kind() != AffineKind::SymbolId || result(i).position() != i) return false;
  return true;
}
bool AffineMap::isMinorIdentity() const {
  return s_ && numDims() >= numResults() &&
         *this == minorIdentity(numDims(), numResults(), context());
}
bool AffineMap::isEmpty() const { return !s_ || (numDims() == 0 && numSymbols() == 0 && numResults() == 0); }
bool AffineMap::isSingleConstant() const {
  return numResults() == 1 && result(0).kind() == AffineKind::Constant;
}
bool AffineMap::isConstant() const {
  for (auto& r : results())
    if (r.kind() != AffineKind::Constant) return false;
  return true;
}
bool AffineMap::isProjectedPermutation(bool allowZero) const {
  if (numSymbols() > 0 || numResults() > numDims()) return false;
  std::vector<bool> seen(numDims(), false);
  for (auto& r : results()) {
    if (r.kind() == AffineKind::DimId) {
      if (seen[r.position()]) return false;
      seen[r.position()] = true;
    } else if (!(allowZero && r == 0)) {
      return false;
    }
  }
  return true;
}
bool AffineMap::isPermutation() const {
  return numDims() == numResults() && isProjectedPermutation();
}
int64_t AffineMap::singleConstantResult() const {
  if (!isSingleConstant()) throw InvalidArgument("map does not have a single constant result");
  return result(0).value();
}
std::vector<int64_t> AffineMap::constantResults() const {
  if (!isConstant()) throw InvalidArgument("map is not constant");
  std::vector<int64_t> v;
  for (auto& r : results()) v.push_back(r.value());
  return v;
}
unsigned AffineMap::dimPosition(unsigned idx) const {
  AffineExpr r = result(idx);
  if (r.kind() != AffineKind::DimId) throw InvalidArgument("result is not a dim expression");
  return r.position();
}
std::optional<unsigned> AffineMap::resultPosition(AffineExpr input) const {
  for (unsigned i = 0; i < numResults(); ++i)
    if (result(i) == input) return i;
  return std::nullopt;
}
std::vector<int64_t> AffineMap::eval(const std::vector<int64_t>& dims,
                                     const std::vector<int64_t>& syms) const {
  std::vector<int64_t> out;
  for (auto& r : results()) out.push_back(r.eval(dims, syms));
  return out;
}
std::string AffineMap::str() const {
  if (!s_) return "<<NULL AFFINE MAP>>";
  std::ostringstream os;
  os << '(';
  for (unsigned i = 0; i < numDims(); ++i) os << (i ? ", " : "") << 'd' << i;
  os << ')';
  if (numSymbols()) {
    os << '[';
    for (unsigned i = 0; i < numSymbols(); ++i) os << (i ? ", " : "") << 's' << i;
    os << ']';
  }
  os << " -> (";
  for (unsigned i = 0; i < numResults(); ++i) os << (i ? ", " : "") << result(i).str();
  os << ')';
  return os.str();
}

// ============================================================================
// Types
// ============================================================================
unsigned Type::bitWidth() const {
  if (isInteger()) return s_->width;
  if (isFloat()) {
    switch (s_->fkind) {
      case FloatKind::F16: case FloatKind::BF16: return 16;
      case FloatKind::F32: return 32;
      case FloatKind::F64: return 64;
      default: return 8;
    }
  }
  if (isIndex()) return 64;
  throw InvalidArgument("type has no bit width: " + str());
}
int64_t Type::dim(int64_t i) const {
  if (i < 0 || i >= rank()) throw std::out_of_range("dimension index out of range");
  return s_->shape[(size_t)i];
}
int64_t Type::numElements() const {
  int64_t n = 1;
  for (int64_t d : s_->shape) n *= d;
  return n;
}
bool Type::hasStaticShape() const {
  for (int64_t d : s_->shape)
    if (d < 0) return false;
  return true;
}
std::optional<MemorySpace> Type::memorySpace() const {
  // Memory space lookup of FriskLayoutAttrs.cpp:1437-1447: no attribute
  // means Local; 0/1/3 name Local/Global/Shared.
  switch (s_->space) {
    case 0: return MemorySpace::Local;
    case 1: return MemorySpace::Global;
    case 3: return MemorySpace::Shared;
    default: return std::nullopt;
  }
}
std::vector<Type> Type::inputs() const {
  std::vector<Type> v;
  for (auto* t : s_->inputs) v.emplace_back(t);
  return v;
}
std::vector<Type> Type::results() const {
  std::vector<Type> v;
  for (auto* t : s_->results) v.emplace_back(t);
  return v;
}

namespace {
const char* floatName(FloatKind k) {
  switch (k) {
    case FloatKind::F16: return "f16";
    case FloatKind::BF16: return "bf16";
    case FloatKind::F32: return "f32";
    case FloatKind::F64: return "f64";
    case FloatKind::E4M3FN: return "f8E4M3FN";
    case FloatKind::E5M2: return "f8E5M2";
  }
  return "?";
}
void printShape(std::ostream& os, const std::vector<int64_t>& shape) {
  for (int64_t d : shape) {
    if (d < 0) os << '?';
    else os << d;
    os << 'x';
  }
}
}  // namespace

std::string Type::str() const {
  if (!s_) return "<<NULL TYPE>>";
  std::ostringstream os;
  switch (s_->kind) {
    case TypeKind::Integer:
      os << (s_->sign == Signedness::Signed ? "si" : s_->sign == Signedness::Unsigned ? "ui" : "i")
         << s_->width;
      break;
    case TypeKind::Float: os << floatName(s_->fkind); break;
    case TypeKind::Index: os << "index"; break;
    case TypeKind::Tensor:
      os << "tensor<";
      printShape(os, s_->shape);
      os << elementType().str() << '>';
      break;
    case TypeKind::MemRef:
      os << "memref<";
      printShape(os, s_->shape);
      os << elementType().str();
      if (s_->layout && !s_->layout.isIdentity()) os << ", affine_map<" << s_->layout.str() << '>';
      if (s_->space != 0) os << ", " << s_->space;
      os << '>';
      break;
    case TypeKind::Function: {
      os << '(';
      for (size_t i = 0; i < s_->inputs.size(); ++i)
        os << (i ? ", " : "") << Type(s_->inputs[i]).str();
      os << ") -> ";
      bool paren = s_->results.size() != 1 || s_->results[0]->kind == TypeKind::Function;
      if (paren) os << '(';
      for (size_t i = 0; i < s_->results.size(); ++i)
        os << (i ? ", " : "") << Type(s_->results[i]).str();
      if (paren) os << ')';
      break;
    }
  }
  return os.str();
}

// ============================================================================
// Float formats
// ============================================================================
namespace {
struct FloatFormat {
  int mant;       // explicit mantissa bits
  int emin;       // minimum normal exponent
  int ebits;
  int bias;
  double maxFinite;
  bool hasInf;
};
FloatFormat formatOf(FloatKind k) {
  switch (k) {
    case FloatKind::F16: return {10, -14, 5, 15, 65504.0, true};
    case FloatKind::BF16: return {7, -126, 8, 127, 3.3895313892515355e38, true};
    case FloatKind::F32: return {23, -126, 8, 127, 3.4028234663852886e38, true};
    case FloatKind::E4M3FN: return {3, -6, 4, 7, 448.0, false};
    case FloatKind::E5M2: return {2, -14, 5, 15, 57344.0, true};
    case FloatKind::F64: break;
  }
  return {52, -1022, 11, 1023, 1.7976931348623157e308, true};
}
}  // namespace

double roundToFloatType(FloatKind k, double v) {
  if (k == FloatKind::F64 || std::isnan(v)) return v;
  const FloatFormat f = formatOf(k);
  if (std::isinf(v)) return f.hasInf ? v : std::nan("");
  if (v == 0.0) return v;
  double a = std::fabs(v);
  int e2;
  std::frexp(a, &e2);  // a = m * 2^e2, m in [0.5, 1)
  int e = std::max(e2 - 1, f.emin);
  double q = std::ldexp(1.0, e - f.mant);
  double r = std::nearbyint(a / q) * q;  // default rounding: nearest, ties to even
  if (r > f.maxFinite) r = f.hasInf ? INFINITY : std::nan("");
  return std::copysign(r, v);
}

uint64_t floatBits(FloatKind k, double v) {
  if (k == FloatKind::F64) {
    uint64_t b;
    std::memcpy(&b, &v, 8);
    return b;
  }
  if (k == FloatKind::F32) {
    float x = (float)v;
    uint32_t b;
    std::memcpy(&b, &x, 4);
    return b;
  }
  const FloatFormat f = formatOf(k);
  const int total = 1 + f.ebits + f.mant;
  const uint64_t sign = std::signbit(v) ? 1ull << (total - 1) : 0;
  const uint64_t expMask = (1ull << f.ebits) - 1;
  if (std::isnan(v)) {
    if (k == FloatKind::E4M3FN) return 0x7F;
    return (expMask << f.mant) | (1ull << (f.mant - 1));
  }
  if (std::isinf(v)) return sign | (expMask << f.mant);
  double a = std::fabs(v);
  if (a == 0.0) return sign;
  int e2;
  std::frexp(a, &e2);
  int e = e2 - 1;
  if (e < f.emin) {  // subnormal
    uint64_t m = (uint64_t)std::ldexp(a, f.mant - f.emin);
    return sign | m;
  }
  uint64_t m = (uint64_t)(std::ldexp(a, f.mant - e)) - (1ull << f.mant);
  return sign | ((uint64_t)(e + f.bias) << f.mant) | m;
}

// ============================================================================
// Attributes
// ============================================================================
namespace {
std::shared_ptr<AttrStorage> newAttr(AttrKind k) {
  auto p = std::make_shared<AttrStorage>();
  p->kind = k;
  return p;
}

std::string formatFloat(FloatKind k, double v) {
  if (std::isfinite(v)) {
    char buf[64];
    std::snprintf(buf, sizeof buf, "%.6e", v);
    if (roundToFloatType(k, std::strtod(buf, nullptr)) == v && std::signbit(v) == (buf[0] == '-'))
      return buf;
    for (int p = 7; p <= 17; ++p) {
      std::snprintf(buf, sizeof buf, "%.*g", p, v);
      if (roundToFloatType(k, std::strtod(buf, nullptr)) == v && std::strchr(buf, '.') &&
          !std::strchr(buf, 'e'))
        return buf;
    }
  }
  // Special or non-round-tripping values: hexadecimal bit pattern.
  const int digits = k == FloatKind::F64 ? 16 : k == FloatKind::F32 ? 8
                     : (k == FloatKind::F16 || k == FloatKind::BF16) ? 4 : 2;
  char buf[32];
  std::snprintf(buf, sizeof buf, "0x%0*llX", digits, (unsigned long long)floatBits(k, v));
  return buf;
}

std::string escapeString(const std::string& s) {
  std::string out = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      out += '\\';
      out += (char)c;
    } else if (c < 0x20 || c >= 0x7f) {
      char b[4];
      std::snprintf(b, sizeof b, "\\%02X", c);
      out += b;
    } else {
      out += (char)c;
    }
  }
  return out + "\"";
}

void printDenseNested(std::ostream& os, const std::vector<int64_t>& shape, size_t dim,
                      size_t& idx, const std::function<void(size_t)>& elem) {
  if (dim == shape.size()) {
    elem(idx++);
    return;
  }
  os << '[';
  for (int64_t i = 0; i < shape[dim]; ++i) {
    if (i) os << ", ";
    printDenseNested(os, shape, dim + 1, idx, elem);
  }
  os << ']';
}
}  // namespace

Attribute Attribute::unit() { return Attribute(newAttr(AttrKind::Unit)); }
Attribute Attribute::boolean(bool v) {
  auto p = newAttr(AttrKind::Bool);
  p->b = v;
  return Attribute(p);
}
Attribute Attribute::integer(Type t, int64_t v) {
  auto p = newAttr(AttrKind::Integer);
  p->type = t;
  p->i = v;
  return Attribute(p);
}
Attribute Attribute::floating(Type t, double v) {
  if (!t.isFloat()) throw InvalidArgument("float attribute needs a float type");
  auto p = newAttr(AttrKind::Float);
  p->type = t;
  p->f = roundToFloatType(t.impl()->fkind, v);
  return Attribute(p);
}
Attribute Attribute::string(std::string s) {
  auto p = newAttr(AttrKind::String);
  p->s = std::move(s);
  return Attribute(p);
}
Attribute Attribute::opaque(std::string text) {
  auto p = newAttr(AttrKind::Opaque);
  p->s = std::move(text);
  return Attribute(p);
}
Attribute Attribute::typeAttr(Type t) {
  auto p = newAttr(AttrKind::TypeA);
  p->type = t;
  return Attribute(p);
}
Attribute Attribute::denseI64(std::vector<int64_t> v) {
  auto p = newAttr(AttrKind::DenseI64Array);
  p->ints = std::move(v);
  return Attribute(p);
}
Attribute Attribute::affineMap(AffineMap m) {
  auto p = newAttr(AttrKind::AffineMapA);
  p->map = m;
  return Attribute(p);
}
Attribute Attribute::memorySpace(MemorySpace s) {
  auto p = newAttr(AttrKind::MemorySpaceA);
  p->i = (int64_t)s;
  return Attribute(p);
}
Attribute Attribute::gemmPolicy(GemmWarpPolicy g) {
  auto p = newAttr(AttrKind::GemmPolicyA);
  p->i = (int64_t)g;
  return Attribute(p);
}
Attribute Attribute::denseFloat(Type tensorTy, std::vector<double> v) {
  if (!tensorTy.isTensor() || !tensorTy.elementType().isFloat())
    throw InvalidArgument("dense float attribute needs a float tensor type");
  if (v.size() != 1 && (int64_t)v.size() != tensorTy.numElements())
    throw InvalidArgument("dense attribute size does not match its tensor type");
  auto p = newAttr(AttrKind::DenseFloat);
  p->type = tensorTy;
  for (double& x : v) x = roundToFloatType(tensorTy.elementType().impl()->fkind, x);
  p->floats = std::move(v);
  return Attribute(p);
}
Attribute Attribute::denseInt(Type tensorTy, std::vector<int64_t> v) {
  if (!tensorTy.isTensor() || !tensorTy.elementType().isInteger())
    throw InvalidArgument("dense integer attribute needs an integer tensor type");
  if (v.size() != 1 && (int64_t)v.size() != tensorTy.numElements())
    throw InvalidArgument("dense attribute size does not match its tensor type");
  auto p = newAttr(AttrKind::DenseInt);
  p->type = tensorTy;
  p->ints = std::move(v);
  return Attribute(p);
}

bool Attribute::operator==(const Attribute& o) const {
  if (p_ == o.p_) return true;
  if (!p_ || !o.p_ || p_->kind != o.p_->kind) return false;
  const AttrStorage &a = *p_, &b = *o.p_;
  switch (a.kind) {
    case AttrKind::Unit: return true;
    case AttrKind::Bool: return a.b == b.b;
    case AttrKind::Integer: return a.type == b.type && a.i == b.i;
    case AttrKind::Float:
      return a.type == b.type && floatBits(a.type.impl()->fkind, a.f) ==
                                     floatBits(b.type.impl()->fkind, b.f);
    case AttrKind::String: case AttrKind::Opaque: return a.s == b.s;
    case AttrKind::TypeA: return a.type == b.type;
    case AttrKind::DenseI64Array: return a.ints == b.ints;
    case AttrKind::AffineMapA: return a.map == b.map;
    case AttrKind::MemorySpaceA: case AttrKind::GemmPolicyA: return a.i == b.i;
    case AttrKind::DenseFloat: return a.type == b.type && a.floats == b.floats;
    case AttrKind::DenseInt: return a.type == b.type && a.ints == b.ints;
  }
  return false;
}

std::string Attribute::str() const {
  if (!p_) return "<<NULL ATTRIBUTE>>";
  const AttrStorage& a = *p_;
  std::ostringstream os;
  switch (a.kind) {
    case AttrKind::Unit: os << "unit"; break;
    case AttrKind::Bool: os << (a.b ? "true" : "false"); break;
    case AttrKind::Integer:
      if (a.type.isInteger(1)) os << (a.i ? "true" : "false");
      else os << a.i << " : " << a.type.str();
      break;
    case AttrKind::Float:
      os << formatFloat(a.type.impl()->fkind, a.f) << " : " << a.type.str();
      break;
    case AttrKind::String: os << escapeString(a.s); break;
    case AttrKind::Opaque: os << a.s; break;
    case AttrKind::TypeA: os << a.type.str(); break;
    case AttrKind::DenseI64Array:
      os << "array<i64";
      for (size_t i = 0; i < a.ints.size(); ++i) os << (i ? ", " : ": ") << a.ints[i];
      os << '>';
      break;
    case AttrKind::AffineMapA: os << "affine_map<" << a.map.str() << '>'; break;
    case AttrKind::MemorySpaceA: {
      const char* n = a.i == 0 ? "Local" : a.i == 1 ? "Global" : a.i == 3 ? "Shared" : "?";
      os << "#frisk.memory_space<" << n << '>';
      break;
    }
    case AttrKind::GemmPolicyA: {
      static const char* names[] = {"Square", "FullRow", "FullCol", "Auto"};
      os << "#frisk.gemm_warp_policy<" << (a.i >= 0 && a.i < 4 ? names[a.i] : "?") << '>';
      break;
    }
    case AttrKind::DenseFloat: case AttrKind::DenseInt: {
      const bool fl = a.kind == AttrKind::DenseFloat;
      const FloatKind fk = fl ? a.type.elementType().impl()->fkind : FloatKind::F32;
      auto elem = [&](size_t i) {
        if (fl) os << formatFloat(fk, a.floats[i]);
        else os << a.ints[i];
      };
      os << "dense<";
      if (isSplat()) {
        elem(0);
      } else {
        size_t idx = 0;
        printDenseNested(os, a.type.shape(), 0, idx, elem);
      }
      os << "> : " << a.type.str();
      break;
    }
  }
  return os.str();
}

// ============================================================================
// Locations
// ============================================================================
std::string Location::str() const {
  if (file.empty()) return "loc(unknown)";
  return "loc(" + escapeString(file) + ":" + std::to_string(line) + ":" + std::to_string(col) + ")";
}

// ============================================================================
// Values
// ============================================================================
void Value::replaceAllUsesWith(Value other) {
  if (other == *this) return;
  std::vector<Operation*> users = v_->users;
  for (Operation* u : users)
    for (unsigned i = 0; i < u->numOperands(); ++i)
      if (u->operands[i] == *this) u->setOperand(i, other);
}

// ============================================================================
// Operations
// ============================================================================
namespace {
void removeUse(ValueImpl* v, Operation* user) {
  auto it = std::find(v->users.begin(), v->users.end(), user);
  if (it != v->users.end()) v->users.erase(it);
}
// Drop the operand uses of `op` and everything nested in it, so that the
// ops can then be destroyed in any order.
void dropAllReferences(Operation* op) {
  op->walk([](Operation* o) { o->dropAllOperands(); });
}
}  // namespace

Operation::~Operation() {
  regions.clear();
  for (Value& v : operands) removeUse(v.impl(), this);
}

Attribute Operation::attr(const std::string& n) const {
  for (auto& a : attrs)
    if (a.name == n) return a.value;
  return Attribute();
}
void Operation::setAttr(const std::string& n, Attribute a) {
  for (auto& x : attrs)
    if (x.name == n) {
      x.value = std::move(a);
      return;
    }
  auto pos = std::lower_bound(attrs.begin(), attrs.end(), n,
                              [](const NamedAttr& x, const std::string& k) { return x.name < k; });
  attrs.insert(pos, NamedAttr{n, std::move(a)});
}
void Operation::removeAttr(const std::string& n) {
  attrs.erase(std::remove_if(attrs.begin(), attrs.end(),
                             [&](const NamedAttr& x) { return x.name == n; }),
              attrs.end());
}
int64_t Operation::intAttr(const std::string& n) const {
  Attribute a = attr(n);
  if (!a || (a.kind() != AttrKind::Integer && a.kind() != AttrKind::MemorySpaceA &&
             a.kind() != AttrKind::GemmPolicyA))
    throw InvalidArgument("'" + name + "' op has no integer attribute " + n);
  return a->i;
}
bool Operation::boolAttr(const std::string& n) const {
  Attribute a = attr(n);
  if (!a || a.kind() != AttrKind::Bool)
    throw InvalidArgument("'" + name + "' op has no bool attribute " + n);
  return a->b;
}
std::string Operation::strAttr(const std::string& n) const {
  Attribute a = attr(n);
  if (!a || a.kind() != AttrKind::String)
    throw InvalidArgument("'" + name + "' op has no string attribute " + n);
  return a->s;
}

void Operation::setOperand(unsigned i, Value v) {
  if (i >= operands.size()) throw std::out_of_range("operand index out of range");
  if (!v) throw InvalidArgument("null operand");
  removeUse(operands[i].impl(), this);
  operands[i] = v;
  v.impl()->users.push_back(this);
}
void Operation::appendOperand(Value v) {
  if (!v) throw InvalidArgument("null operand");
  operands.push_back(v);
  v.impl()->users.push_back(this);
}
void Operation::setOperands(const std::vector<Value>& vs) {
  dropAllOperands();
  for (auto& v : vs) appendOperand(v);
}
void Operation::dropAllOperands() {
  for (Value& v : operands) removeUse(v.impl(), this);
  operands.clear();
}
Value Operation::addResult(Type t) {
  auto v = std::make_unique<ValueImpl>();
  v->type = t;
  v->def = this;
  v->index = (unsigned)results.size();
  results.push_back(std::move(v));
  return Value(results.back().get());
}
Region* Operation::addRegion() {
  regions.push_back(std::make_unique<Region>());
  regions.back()->parent = this;
  return regions.back().get();
}
Block* Operation::body(unsigned r) const {
  if (r >= regions.size()) return nullptr;
  return regions[r]->front();
}
Operation* Operation::parentOp() const { return parent ? parent->parentOp() : nullptr; }
bool Operation::isAncestorOf(const Operation* other) const {
  for (const Operation* p = other; p; p = p->parentOp())
    if (p == this) return true;
  return false;
}
bool Operation::isBeforeInBlock(const Operation* other) const {
  if (!parent || parent != other->parent) throw InvalidArgument("ops are not in the same block");
  for (auto it = self; it != parent->ops.end(); ++it)
    if (it->get() == other) return it->get() != this;
  return false;
}
bool Operation::isTerminator() const {
  return name == "frisk.end" || name == "scf.yield" || name == "func.return";
}

std::unique_ptr<Operation> Operation::remove() {
  if (parent) {
    std::unique_ptr<Operation> up = std::move(*self);
    parent->ops.erase(self);
    up->parent = nullptr;
    return up;
  }
  return ctx->release(this);
}

void Operation::erase() {
  for (auto& r : results)
    if (!r->users.empty())
      throw InvalidArgument("'" + name + "' op cannot be erased while its results have uses");
  std::unique_ptr<Operation> up = remove();
  dropAllReferences(up.get());
}

void Operation::walk(const std::function<void(Operation*)>& fn) {
  for (auto& r : regions) r->walk(fn);
  fn(this);
}

// ============================================================================
// Blocks and regions
// ============================================================================
Block::~Block() {
  for (auto& op : ops) dropAllReferences(op.get());
  ops.clear();
}
Value Block::addArgument(Type t) {
  auto v = std::make_unique<ValueImpl>();
  v->type = t;
  v->owner = this;
  v->index = (unsigned)args.size();
  args.push_back(std::move(v));
  return Value(args.back().get());
}
Operation* Block::parentOp() const { return parent ? parent->parent : nullptr; }
Operation* Block::terminator() const {
  Operation* b = back();
  return (b && b->isTerminator()) ? b : nullptr;
}
Operation* Block::insert(std::list<std::unique_ptr<Operation>>::iterator pos,
                         std::unique_ptr<Operation> op) {
  op->parent = this;
  Operation* raw = op.get();
  raw->self = ops.insert(pos, std::move(op));
  return raw;
}
Operation* Block::findAncestorOpInBlock(Operation* op) const {
  for (Operation* p = op; p; p = p->parentOp())
    if (p->parent == this) return p;
  return nullptr;
}
void Block::walk(const std::function<void(Operation*)>& fn) {
  for (auto it = ops.begin(); it != ops.end();) {
    Operation* op = (it++)->get();  // tolerate erasure of the visited op
    op->walk(fn);
  }
}

Block* Region::pushBack(std::unique_ptr<Block> b) {
  b->parent = this;
  blocks.push_back(std::move(b));
  return blocks.back().get();
}
Region* Region::parentRegion() const {
  return (parent && parent->parent) ? parent->parent->parent : nullptr;
}
void Region::walk(const std::function<void(Operation*)>& fn) {
  for (auto& b : blocks) b->walk(fn);
}
void Region::takeBody(Region& other) {
  if (!blocks.empty()) throw InvalidArgument("takeBody into a non-empty region");
  blocks.splice(blocks.end(), other.blocks);
  for (auto& b : blocks) b->parent = this;
}

// ============================================================================
// Context
// ============================================================================
Context::Context() = default;
Context::~Context() {
  for (auto& op : detached_) dropAllReferences(op.get());
  for (auto& b : detachedBlocks_)
    for (auto& op : b->ops) dropAllReferences(op.get());
  detached_.clear();
  detachedBlocks_.clear();
}

Block* Context::adoptBlock(std::unique_ptr<Block> b) {
  b->parent = nullptr;
  detachedBlocks_.push_back(std::move(b));
  return detachedBlocks_.back().get();
}
std::unique_ptr<Block> Context::releaseBlock(Block* b) {
  for (auto it = detachedBlocks_.begin(); it != detachedBlocks_.end(); ++it)
    if (it->get() == b) {
      std::unique_ptr<Block> up = std::move(*it);
      detachedBlocks_.erase(it);
      return up;
    }
  return nullptr;
}

const TypeStorage* Context::uniqueType(TypeStorage&& t) {
  t.ctx = this;
  // Key: the printed form is unique per type (layout maps are uniqued too).
  std::ostringstream key;
  key << (int)t.kind << '|' << t.width << '|' << (int)t.sign << '|' << (int)t.fkind << '|'
      << t.elem << '|' << t.layout.impl() << '|' << t.space << '|';
  for (auto d : t.shape) key << d << ',';
  key << '|';
  for (auto* p : t.inputs) key << p << ',';
  key << '|';
  for (auto* p : t.results) key << p << ',';
  auto it = typeIndex_.find(key.str());
  if (it != typeIndex_.end()) return it->second;
  types_.push_back(std::move(t));
  typeIndex_.emplace(key.str(), &types_.back());
  return &types_.back();
}

Type Context::integer(unsigned width, Signedness s) {
  if (width == 0) throw InvalidArgument("integer width must be positive");
  TypeStorage t;
  t.kind = TypeKind::Integer;
  t.width = width;
  t.sign = s;
  return Type(uniqueType(std::move(t)));
}
Type Context::floatTy(FloatKind k) {
  TypeStorage t;
  t.kind = TypeKind::Float;
  t.fkind = k;
  return Type(uniqueType(std::move(t)));
}
Type Context::index() {
  TypeStorage t;
  t.kind = TypeKind::Index;
  return Type(uniqueType(std::move(t)));
}
Type Context::memref(const std::vector<int64_t>& shape, Type elem, AffineMap layout, int64_t space) {
  if (!elem) throw InvalidArgument("memref needs an element type");
  for (int64_t d : shape)
    if (d < -1) throw InvalidArgument("memref extents must be non-negative or dynamic");
  if (layout && layout.numDims() != shape.size())
    throw InvalidArgument("memref layout map must have one dim per memref dimension");
  TypeStorage t;
  t.kind = TypeKind::MemRef;
  t.shape = shape;
  t.elem = elem.impl();
  // An identity layout is the default layout.
  t.layout = (layout && !layout.isIdentity()) ? layout : AffineMap();
  t.space = space;
  return Type(uniqueType(std::move(t)));
}
Type Context::tensor(const std::vector<int64_t>& shape, Type elem) {
  if (!elem) throw InvalidArgument("tensor needs an element type");
  TypeStorage t;
  t.kind = TypeKind::Tensor;
  t.shape = shape;
  t.elem = elem.impl();
  return Type(uniqueType(std::move(t)));
}
Type Context::function(const std::vector<Type>& ins, const std::vector<Type>& outs) {
  TypeStorage t;
  t.kind = TypeKind::Function;
  for (auto& x : ins) t.inputs.push_back(x.impl());
  for (auto& x : outs) t.results.push_back(x.impl());
  return Type(uniqueType(std::move(t)));
}

const AffineExprStorage* Context::uniqueExpr(AffineKind k, int64_t v, const AffineExprStorage* l,
                                             const AffineExprStorage* r) {
  auto key = std::make_tuple((int)k, v, (const void*)l, (const void*)r);
  auto it = exprIndex_.find(key);
  if (it != exprIndex_.end()) return it->second;
  exprs_.push_back(AffineExprStorage{this, k, v, l, r});
  exprIndex_.emplace(key, &exprs_.back());
  return &exprs_.back();
}

const AffineMapStorage* Context::uniqueMap(unsigned dims, unsigned syms,
                                           const std::vector<AffineExpr>& results) {
  std::ostringstream key;
  key << dims << '|' << syms << '|';
  for (auto& r : results) key << r.impl() << ',';
  auto it = mapIndex_.find(key.str());
  if (it != mapIndex_.end()) return it->second;
  maps_.push_back(AffineMapStorage{this, dims, syms, results});
  mapIndex_.emplace(key.str(), &maps_.back());
  return &maps_.back();
}

Operation* Context::adopt(std::unique_ptr<Operation> op) {
  op->parent = nullptr;
  detached_.push_back(std::move(op));
  return detached_.back().get();
}
std::unique_ptr<Operation> Context::release(Operation* op) {
  for (auto it = detached_.begin(); it != detached_.end(); ++it)
    if (it->get() == op) {
      std::unique_ptr<Operation> up = std::move(*it);
      detached_.erase(it);
      return up;
    }
  return nullptr;
}
bool Context::isDetached(const Operation* op) const {
  for (auto& d : detached_)
    if (d.get() == op) return true;
  return false;
}

// ============================================================================
// Builder
// ============================================================================
std::unique_ptr<Operation> makeOp(Context* ctx, const std::string& name, Location loc,
                                  const std::vector<Value>& operands,
                                  const std::vector<Type>& resultTypes,
                                  std::vector<NamedAttr> attrs, unsigned numRegions) {
  auto op = std::make_unique<Operation>();
  op->ctx = ctx;
  op->name = name;
  op->loc = std::move(loc);
  for (auto& v : operands) op->appendOperand(v);
  for (auto& t : resultTypes) op->addResult(t);
  for (auto& a : attrs) op->setAttr(a.name, a.value);
  for (unsigned i = 0; i < numRegions; ++i) op->addRegion();
  return op;
}

Operation* Builder::insert(std::unique_ptr<Operation> op) {
  if (ip_.block) return ip_.block->insert(ip_.pos, std::move(op));
  return ctx_->adopt(std::move(op));
}
Operation* Builder::create(const std::string& name, const std::vector<Value>& operands,
                           const std::vector<Type>& resultTypes, std::vector<NamedAttr> attrs,
                           unsigned numRegions) {
  return insert(makeOp(ctx_, name, loc_, operands, resultTypes, std::move(attrs), numRegions));
}

std::unique_ptr<Operation> cloneOp(Operation* op, std::unordered_map<ValueImpl*, Value>& map) {
  std::vector<Value> ops;
  for (auto& v : op->operands) {
    auto it = map.find(v.impl());
    ops.push_back(it == map.end() ? v : it->second);
  }
  std::vector<Type> rt;
  for (auto& r : op->results) rt.push_back(r->type);
  auto c = makeOp(op->ctx, op->name, op->loc, ops, rt, op->attrs, 0);
  for (unsigned i = 0; i < op->numResults(); ++i) map[op->results[i].get()] = c->result(i);
  for (auto& r : op->regions) {
    Region* nr = c->addRegion();
    for (auto& b : r->blocks) {
      Block* nb = nr->emplaceBlock();
      for (auto& a : b->args) map[a.get()] = nb->addArgument(a->type);
    }
    auto bit = nr->blocks.begin();
    for (auto& b : r->blocks) {
      for (auto& o : b->ops) (*bit)->pushBack(cloneOp(o.get(), map));
      ++bit;
    }
  }
  return c;
}

Operation* Builder::clone(Operation* op) {
  std::unordered_map<ValueImpl*, Value> map;
  return insert(cloneOp(op, map));
}

}  // namespace fir
