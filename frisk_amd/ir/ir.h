// Host-side tile IR for the Frisk GEMM / attention path.
//
// A compact, MLIR-shaped IR (operations with operands, results, attributes
// and regions of blocks) that carries exactly what the reference builds
// through its pybind11 `frisk_ffi.ir` module (ffi/ir.cpp): the `frisk`
// dialect ops (kernel, parallel, block, for, gemm, alloc_buffer, copy, fill,
// reduce; include/Dialect/Frisk/IR/FriskOps.td), the tensor-form layout ops
// the normalizer produces (mma, reduce_tensor, tile_load, tile_store,
// layout_view; FriskLayoutOps.td) and the few builtin/arith/scf/func ops they
// need.  There is no MLIR here: types, affine expressions and maps are
// interned in a Context, values keep use lists, and ops own their regions.
//
// Ownership follows MLIR: a Block owns its operations and arguments, a
// Region owns its blocks, an Operation owns its regions and results.  An
// operation created without an insertion block (modules, kernels created
// before they are pushed into a module) is owned by the Context until it is
// inserted somewhere.  Handles (Type, Value, Operation*) are non-owning.
#pragma once

#include <cstdint>
#include <deque>
#include <functional>
#include <list>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace fir {

class Context;
struct Operation;
struct Block;
struct Region;

// ----------------------------------------------------------------------------
// Affine expressions and maps (mlir/IR/AffineExpr.h semantics, own code).
// ----------------------------------------------------------------------------
// Kind numbering follows the reference's exposed AffineExprKind enum
// (ffi/ir.cpp:736-746): binary kinds first, LAST_AFFINE_BINARY_OP = CeilDiv.
enum class AffineKind : int { Add = 0, Mul, Mod, FloorDiv, CeilDiv, Constant, DimId, SymbolId };
constexpr int kLastAffineBinaryOp = static_cast<int>(AffineKind::CeilDiv);

struct AffineExprStorage {
  Context* ctx;
  AffineKind kind;
  int64_t value;  // constant value or dim/symbol position
  const AffineExprStorage* lhs;
  const AffineExprStorage* rhs;
};

class AffineExpr {
 public:
  AffineExpr() = default;
  explicit AffineExpr(const AffineExprStorage* s) : s_(s) {}
  explicit operator bool() const { return s_ != nullptr; }
  bool operator==(const AffineExpr& o) const { return s_ == o.s_; }
  bool operator!=(const AffineExpr& o) const { return s_ != o.s_; }
  bool operator==(int64_t v) const;
  const AffineExprStorage* impl() const { return s_; }
  Context* context() const;
  AffineKind kind() const;
  bool isBinary() const { return s_ && static_cast<int>(s_->kind) <= kLastAffineBinaryOp; }
  AffineExpr lhs() const { return AffineExpr(s_->lhs); }
  AffineExpr rhs() const { return AffineExpr(s_->rhs); }
  int64_t value() const { return s_->value; }      // Constant
  unsigned position() const { return (unsigned)s_->value; }  // DimId / SymbolId

  bool isSymbolicOrConstant() const;
  bool isPureAffine() const;
  int64_t largestKnownDivisor() const;
  bool isMultipleOf(int64_t f) const;
  bool isFunctionOfDim(unsigned pos) const;
  bool isFunctionOfSymbol(unsigned pos) const;
  AffineExpr replaceDimsAndSymbols(const std::vector<AffineExpr>& dims,
                                   const std::vector<AffineExpr>& syms) const;
  AffineExpr replace(const std::map<const AffineExprStorage*, AffineExpr>& m) const;
  AffineExpr shiftDims(unsigned numDims, unsigned shift, unsigned offset = 0) const;
  AffineExpr shiftSymbols(unsigned numSyms, unsigned shift, unsigned offset = 0) const;
  // Evaluate with concrete dim / symbol values (floor semantics for div/mod).
  int64_t eval(const std::vector<int64_t>& dims, const std::vector<int64_t>& syms = {}) const;
  std::string str() const;

 private:
  const AffineExprStorage* s_ = nullptr;
};

AffineExpr operator+(AffineExpr a, AffineExpr b);
AffineExpr operator+(AffineExpr a, int64_t b);
AffineExpr operator*(AffineExpr a, AffineExpr b);
AffineExpr operator*(AffineExpr a, int64_t b);
AffineExpr operator-(AffineExpr a);
AffineExpr operator-(AffineExpr a, AffineExpr b);
AffineExpr operator-(AffineExpr a, int64_t b);
AffineExpr operator%(AffineExpr a, AffineExpr b);
AffineExpr operator%(AffineExpr a, uint64_t b);
AffineExpr floorDiv(AffineExpr a, AffineExpr b);
AffineExpr floorDiv(AffineExpr a, uint64_t b);
AffineExpr ceilDiv(AffineExpr a, AffineExpr b);
AffineExpr ceilDiv(AffineExpr a, uint64_t b);

AffineExpr getAffineDimExpr(unsigned pos, Context* ctx);
AffineExpr getAffineSymbolExpr(unsigned pos, Context* ctx);
AffineExpr getAffineConstantExpr(int64_t v, Context* ctx);
AffineExpr getAffineBinaryOpExpr(AffineKind kind, AffineExpr lhs, AffineExpr rhs);

struct AffineMapStorage {
  Context* ctx;
  unsigned numDims, numSymbols;
  std::vector<AffineExpr> results;
};

class AffineMap {
 public:
  AffineMap() = default;
  explicit AffineMap(const AffineMapStorage* s) : s_(s) {}
  explicit operator bool() const { return s_ != nullptr; }
  bool operator==(const AffineMap& o) const { return s_ == o.s_; }
  bool operator!=(const AffineMap& o) const { return s_ != o.s_; }
  const AffineMapStorage* impl() const { return s_; }

  static AffineMap get(Context* ctx);  // () -> ()
  static AffineMap get(unsigned dims, unsigned syms, Context* ctx);
  static AffineMap get(unsigned dims, unsigned syms, AffineExpr result);
  static AffineMap get(unsigned dims, unsigned syms, const std::vector<AffineExpr>& results,
                       Context* ctx);
  static AffineMap constantMap(int64_t v, Context* ctx);
  static AffineMap multiDimIdentity(unsigned dims, Context* ctx);
  static AffineMap minorIdentity(unsigned dims, unsigned results, Context* ctx);
  static AffineMap permutation(const std::vector<unsigned>& perm, Context* ctx);

  Context* context() const { return s_ ? s_->ctx : nullptr; }
  unsigned numDims() const { return s_ ? s_->numDims : 0; }
  unsigned numSymbols() const { return s_ ? s_->numSymbols : 0; }
  unsigned numResults() const { return s_ ? (unsigned)s_->results.size() : 0; }
  unsigned numInputs() const { return numDims() + numSymbols(); }
  const std::vector<AffineExpr>& results() const;
  AffineExpr result(unsigned i) const;
  bool isIdentity() const;
  bool isSymbolIdentity() const;
  bool isMinorIdentity() const;
  bool isEmpty() const;
  bool isSingleConstant() const;
  bool isConstant() const;
  bool isPermutation() const;
  bool isProjectedPermutation(bool allowZeroInResults = false) const;
  int64_t singleConstantResult() const;
  std::vector<int64_t> constantResults() const;
  unsigned dimPosition(unsigned idx) const;
  std::optional<unsigned> resultPosition(AffineExpr input) const;
  std::vector<int64_t> eval(const std::vector<int64_t>& dims,
                            const std::vector<int64_t>& syms = {}) const;
  std::string str() const;

 private:
  const AffineMapStorage* s_ = nullptr;
};

// ----------------------------------------------------------------------------
// Types.
// ----------------------------------------------------------------------------
enum class TypeKind : uint8_t { Integer, Float, Index, MemRef, Tensor, Function };
enum class FloatKind : uint8_t { F16, BF16, F32, F64, E4M3FN, E5M2 };
enum class Signedness : uint8_t { Signless, Signed, Unsigned };

// Memory spaces of include/Dialect/Frisk/IR/FriskEnums.td:6-8.
enum class MemorySpace : int32_t { Local = 0, Global = 1, Shared = 3 };
// GEMM warp partition policies of FriskEnums.td:17-26.
enum class GemmWarpPolicy : int32_t { Square = 0, FullRow = 1, FullCol = 2, Auto = 3 };

struct TypeStorage {
  Context* ctx;
  TypeKind kind;
  unsigned width = 0;
  Signedness sign = Signedness::Signless;
  FloatKind fkind = FloatKind::F32;
  std::vector<int64_t> shape;
  const TypeStorage* elem = nullptr;
  AffineMap layout;       // memref layout map (null = identity)
  int64_t space = 0;      // memref memory space integer (0 = default = Local)
  std::vector<const TypeStorage*> inputs, results;  // function
};

class Type {
 public:
  Type() = default;
  explicit Type(const TypeStorage* s) : s_(s) {}
  explicit operator bool() const { return s_ != nullptr; }
  bool operator==(const Type& o) const { return s_ == o.s_; }
  bool operator!=(const Type& o) const { return s_ != o.s_; }
  const TypeStorage* impl() const { return s_; }
  Context* context() const { return s_ ? s_->ctx : nullptr; }
  TypeKind kind() const { return s_->kind; }

  bool isInteger() const { return s_ && s_->kind == TypeKind::Integer; }
  bool isInteger(unsigned w) const { return isInteger() && s_->width == w; }
  bool isSignlessInteger() const { return isInteger() && s_->sign == Signedness::Signless; }
  bool isSignlessInteger(unsigned w) const { return isSignlessInteger() && s_->width == w; }
  bool isSignedInteger() const { return isInteger() && s_->sign == Signedness::Signed; }
  bool isUnsignedInteger() const { return isInteger() && s_->sign == Signedness::Unsigned; }
  bool isFloat() const { return s_ && s_->kind == TypeKind::Float; }
  bool isFloat(FloatKind k) const { return isFloat() && s_->fkind == k; }
  bool isF16() const { return isFloat(FloatKind::F16); }
  bool isBF16() const { return isFloat(FloatKind::BF16); }
  bool isF32() const { return isFloat(FloatKind::F32); }
  bool isF64() const { return isFloat(FloatKind::F64); }
  bool isIndex() const { return s_ && s_->kind == TypeKind::Index; }
  bool isMemRef() const { return s_ && s_->kind == TypeKind::MemRef; }
  bool isTensor() const { return s_ && s_->kind == TypeKind::Tensor; }
  bool isShaped() const { return isMemRef() || isTensor(); }
  bool isFunction() const { return s_ && s_->kind == TypeKind::Function; }
  bool isIntOrFloat() const { return isInteger() || isFloat(); }

  unsigned bitWidth() const;  // integer / float element width
  // Shaped types.
  const std::vector<int64_t>& shape() const { return s_->shape; }
  int64_t rank() const { return (int64_t)s_->shape.size(); }
  int64_t dim(int64_t i) const;
  int64_t numElements() const;
  bool hasStaticShape() const;
  Type elementType() const { return Type(s_->elem); }
  AffineMap layout() const { return s_->layout; }
  int64_t memorySpaceInt() const { return s_->space; }
  std::optional<MemorySpace> memorySpace() const;  // frisk memory space, if recognised
  // Function types.
  std::vector<Type> inputs() const;
  std::vector<Type> results() const;

  std::string str() const;

 private:
  const TypeStorage* s_ = nullptr;
};

// ----------------------------------------------------------------------------
// Attributes (value-semantic).
// ----------------------------------------------------------------------------
enum class AttrKind : uint8_t {
  Unit, Bool, Integer, Float, String, TypeA, DenseI64Array, AffineMapA, MemorySpaceA,
  GemmPolicyA, DenseFloat, DenseInt,
  Opaque  // a dialect attribute kept as its textual form, printed verbatim
};

struct AttrStorage {
  AttrKind kind = AttrKind::Unit;
  bool b = false;
  int64_t i = 0;
  double f = 0.0;
  Type type;  // integer/float/dense element type, or the TypeAttr value
  std::string s;
  std::vector<int64_t> ints;
  std::vector<double> floats;
  AffineMap map;
};

class Attribute {
 public:
  Attribute() = default;
  explicit Attribute(std::shared_ptr<const AttrStorage> p) : p_(std::move(p)) {}
  explicit operator bool() const { return p_ != nullptr; }
  const AttrStorage* operator->() const { return p_.get(); }
  AttrKind kind() const { return p_->kind; }
  bool operator==(const Attribute& o) const;
  bool operator!=(const Attribute& o) const { return !(*this == o); }
  std::string str() const;

  static Attribute unit();
  static Attribute boolean(bool v);
  static Attribute integer(Type t, int64_t v);
  // Float attributes hold the value rounded to the element type (round to
  // nearest even, saturating fp8 kinds like their finite-only encodings).
  static Attribute floating(Type t, double v);
  static Attribute string(std::string s);
  static Attribute opaque(std::string text);
  static Attribute typeAttr(Type t);
  static Attribute denseI64(std::vector<int64_t> v);
  static Attribute affineMap(AffineMap m);
  static Attribute memorySpace(MemorySpace s);
  static Attribute gemmPolicy(GemmWarpPolicy p);
  static Attribute denseFloat(Type tensorTy, std::vector<double> v);  // size 1 = splat
  static Attribute denseInt(Type tensorTy, std::vector<int64_t> v);

  bool isSplat() const { return (p_->kind == AttrKind::DenseFloat && p_->floats.size() == 1) ||
                                (p_->kind == AttrKind::DenseInt && p_->ints.size() == 1); }

 private:
  std::shared_ptr<const AttrStorage> p_;
};

// Round `v` to the value set of float type `t` (f16/bf16/f32/f64/e4m3fn/e5m2).
double roundToFloatType(FloatKind k, double v);
// Bit pattern of `v` (already representable) in float type `k`.
uint64_t floatBits(FloatKind k, double v);

// ----------------------------------------------------------------------------
// Locations.
// ----------------------------------------------------------------------------
struct Location {
  std::string file;  // empty = unknown
  int line = 0, col = 0;
  std::string str() const;
};

// ----------------------------------------------------------------------------
// Values, operations, blocks, regions.
// ----------------------------------------------------------------------------
struct ValueImpl {
  Type type;
  Operation* def = nullptr;   // defining op (op result)
  Block* owner = nullptr;     // owning block (block argument)
  unsigned index = 0;         // result / argument number
  std::vector<Operation*> users;  // one entry per use
};

class Value {
 public:
  Value() = default;
  explicit Value(ValueImpl* v) : v_(v) {}
  explicit operator bool() const { return v_ != nullptr; }
  bool operator==(const Value& o) const { return v_ == o.v_; }
  bool operator!=(const Value& o) const { return v_ != o.v_; }
  bool operator<(const Value& o) const { return v_ < o.v_; }
  ValueImpl* impl() const { return v_; }
  Type type() const { return v_->type; }
  void setType(Type t) { v_->type = t; }
  Operation* definingOp() const { return v_->def; }
  Block* ownerBlock() const { return v_->owner; }
  bool isBlockArgument() const { return v_->owner != nullptr; }
  unsigned index() const { return v_->index; }
  const std::vector<Operation*>& users() const { return v_->users; }
  bool useEmpty() const { return v_->users.empty(); }
  void replaceAllUsesWith(Value other);
  Context* context() const { return v_->type.context(); }

 private:
  ValueImpl* v_ = nullptr;
};

struct ValueHash {
  size_t operator()(const Value& v) const { return std::hash<void*>()(v.impl()); }
};

struct NamedAttr {
  std::string name;
  Attribute value;
};

struct Operation {
  std::string name;
  Location loc;
  std::vector<Value> operands;
  std::vector<std::unique_ptr<ValueImpl>> results;
  std::vector<NamedAttr> attrs;  // kept sorted by name
  std::vector<std::unique_ptr<Region>> regions;
  Block* parent = nullptr;
  std::list<std::unique_ptr<Operation>>::iterator self;  // position in parent block
  Context* ctx = nullptr;

  Operation() = default;
  Operation(const Operation&) = delete;
  Operation& operator=(const Operation&) = delete;
  ~Operation();

  // Attributes.
  Attribute attr(const std::string& n) const;
  bool hasAttr(const std::string& n) const { return (bool)attr(n); }
  void setAttr(const std::string& n, Attribute a);
  void removeAttr(const std::string& n);
  int64_t intAttr(const std::string& n) const;
  bool boolAttr(const std::string& n) const;
  std::string strAttr(const std::string& n) const;

  // Operands / results.
  unsigned numOperands() const { return (unsigned)operands.size(); }
  Value operand(unsigned i) const { return operands.at(i); }
  void setOperand(unsigned i, Value v);
  void appendOperand(Value v);
  void setOperands(const std::vector<Value>& vs);
  void dropAllOperands();
  unsigned numResults() const { return (unsigned)results.size(); }
  Value result(unsigned i) const { return Value(results.at(i).get()); }
  Value addResult(Type t);

  // Structure.
  unsigned numRegions() const { return (unsigned)regions.size(); }
  Region& region(unsigned i) const { return *regions.at(i); }
  Region* addRegion();
  Block* body(unsigned region = 0) const;  // first block of a region
  Operation* parentOp() const;
  bool isAncestorOf(const Operation* other) const;
  bool isBeforeInBlock(const Operation* other) const;
  bool isTerminator() const;

  // Detach from the parent block (ownership returns to the caller) / erase.
  std::unique_ptr<Operation> remove();
  void erase();
  void walk(const std::function<void(Operation*)>& fn);  // post-order like MLIR

  bool is(const char* n) const { return name == n; }
};

struct Block {
  std::vector<std::unique_ptr<ValueImpl>> args;
  std::list<std::unique_ptr<Operation>> ops;
  Region* parent = nullptr;

  Block() = default;
  Block(const Block&) = delete;
  Block& operator=(const Block&) = delete;
  ~Block();
  unsigned numArguments() const { return (unsigned)args.size(); }
  Value argument(unsigned i) const { return Value(args.at(i).get()); }
  Value addArgument(Type t);
  Operation* parentOp() const;
  Operation* terminator() const;
  bool empty() const { return ops.empty(); }
  Operation* front() const { return ops.empty() ? nullptr : ops.front().get(); }
  Operation* back() const { return ops.empty() ? nullptr : ops.back().get(); }
  // Insert an op (taking ownership) before `pos`.
  Operation* insert(std::list<std::unique_ptr<Operation>>::iterator pos,
                    std::unique_ptr<Operation> op);
  Operation* pushBack(std::unique_ptr<Operation> op) { return insert(ops.end(), std::move(op)); }
  // Ancestor of `op` that sits directly in this block, or nullptr.
  Operation* findAncestorOpInBlock(Operation* op) const;
  void walk(const std::function<void(Operation*)>& fn);
};

struct Region {
  std::list<std::unique_ptr<Block>> blocks;
  Operation* parent = nullptr;

  Region() = default;
  Region(const Region&) = delete;
  Region& operator=(const Region&) = delete;

  bool empty() const { return blocks.empty(); }
  size_t size() const { return blocks.size(); }
  Block* front() const { return blocks.empty() ? nullptr : blocks.front().get(); }
  Block* pushBack(std::unique_ptr<Block> b);
  Block* emplaceBlock() { return pushBack(std::make_unique<Block>()); }
  Region* parentRegion() const;
  void walk(const std::function<void(Operation*)>& fn);
  // Move all blocks of `other` into this (empty) region.
  void takeBody(Region& other);
};

// ----------------------------------------------------------------------------
// Context: type / affine uniquing and ownership of detached operations.
// ----------------------------------------------------------------------------
class Context {
 public:
  Context();
  ~Context();
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;

  // Types.
  Type integer(unsigned width, Signedness s = Signedness::Signless);
  Type floatTy(FloatKind k);
  Type index();
  Type memref(const std::vector<int64_t>& shape, Type elem, AffineMap layout = AffineMap(),
              int64_t space = 0);
  Type tensor(const std::vector<int64_t>& shape, Type elem);
  Type function(const std::vector<Type>& ins, const std::vector<Type>& outs);

  // Affine uniquing.
  const AffineExprStorage* uniqueExpr(AffineKind k, int64_t v, const AffineExprStorage* l,
                                      const AffineExprStorage* r);
  const AffineMapStorage* uniqueMap(unsigned dims, unsigned syms,
                                    const std::vector<AffineExpr>& results);

  // Detached operations.
  Operation* adopt(std::unique_ptr<Operation> op);
  std::unique_ptr<Operation> release(Operation* op);  // nullptr if not detached
  bool isDetached(const Operation* op) const;
  // Detached blocks (created before they are placed in a region).
  Block* adoptBlock(std::unique_ptr<Block> b);
  std::unique_ptr<Block> releaseBlock(Block* b);  // nullptr if not detached

  void disableMultithreading() { multithreading_ = false; }
  bool multithreading() const { return multithreading_; }
  bool dialectsLoaded = false;

 private:
  const TypeStorage* uniqueType(TypeStorage&& t);
  std::deque<TypeStorage> types_;
  std::unordered_map<std::string, const TypeStorage*> typeIndex_;
  std::deque<AffineExprStorage> exprs_;
  std::map<std::tuple<int, int64_t, const void*, const void*>, const AffineExprStorage*> exprIndex_;
  std::deque<AffineMapStorage> maps_;
  std::map<std::string, const AffineMapStorage*> mapIndex_;
  std::list<std::unique_ptr<Operation>> detached_;
  std::list<std::unique_ptr<Block>> detachedBlocks_;
  bool multithreading_ = true;
};

// Create an unattached op.  The caller inserts it (Builder::insert) or hands
// it to Context::adopt.
std::unique_ptr<Operation> makeOp(Context* ctx, const std::string& name, Location loc,
                                  const std::vector<Value>& operands,
                                  const std::vector<Type>& resultTypes,
                                  std::vector<NamedAttr> attrs = {}, unsigned numRegions = 0);

// ----------------------------------------------------------------------------
// Builder: an insertion point plus the current location.
// ----------------------------------------------------------------------------
struct InsertPoint {
  Block* block = nullptr;
  std::list<std::unique_ptr<Operation>>::iterator pos;
  bool isSet() const { return block != nullptr; }
};

class Builder {
 public:
  explicit Builder(Context* ctx) : ctx_(ctx) {}
  Context* context() const { return ctx_; }

  void setInsertionPointToStart(Block* b) { ip_ = {b, b->ops.begin()}; }
  void setInsertionPointToEnd(Block* b) { ip_ = {b, b->ops.end()}; }
  void setInsertionPoint(Operation* op) { ip_ = {op->parent, op->self}; }
  void setInsertionPointAfter(Operation* op) { ip_ = {op->parent, std::next(op->self)}; }
  void clearInsertionPoint() { ip_ = {}; }
  Block* insertionBlock() const { return ip_.block; }
  InsertPoint saveInsertionPoint() const { return ip_; }
  void restoreInsertionPoint(InsertPoint ip) { ip_ = ip; }

  void setLoc(Location l) { loc_ = std::move(l); }
  const Location& loc() const { return loc_; }

  // Insert at the insertion point, or hand to the context when there is none.
  Operation* insert(std::unique_ptr<Operation> op);
  Operation* create(const std::string& name, const std::vector<Value>& operands,
                    const std::vector<Type>& resultTypes, std::vector<NamedAttr> attrs = {},
                    unsigned numRegions = 0);
  Operation* clone(Operation* op);

 private:
  Context* ctx_;
  InsertPoint ip_;
  Location loc_;
};

// Deep copy (operands remapped through `map` where present).
std::unique_ptr<Operation> cloneOp(Operation* op, std::unordered_map<ValueImpl*, Value>& map);

// ----------------------------------------------------------------------------
// Printing (MLIR-style textual form) and verification.
// ----------------------------------------------------------------------------
struct PrintOptions {
  bool debugInfo = false;  // print `loc(...)` after each op
};
std::string printOp(Operation* op, PrintOptions opts = {});
// The operations of a block, one per line (names relative to its top op).
std::string printBlock(Block* b, PrintOptions opts = {});
// Operand-style name of `v` (`%arg0`, `%3`) within its top-level op.
std::string printValueAsOperand(Value v);

// Verify `op` and everything nested in it.  On failure returns false and
// stores the first diagnostic ("'<op>' op <message>") in `*diag`.
bool verify(Operation* op, std::string* diag);

// Error type mapped to Python ValueError by the bindings.
struct InvalidArgument : std::invalid_argument {
  using std::invalid_argument::invalid_argument;
};

}  // namespace fir
