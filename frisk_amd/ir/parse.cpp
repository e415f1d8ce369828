// Recursive-descent parser of the textual tile IR (see parse.h).  Each custom
// form below is the inverse of the matching routine of print.cpp; operations
// in MLIR's generic form are built as written.  Attributes elided by a custom
// form are rebuilt as the builders of ops.cpp set them (alloc_buffer's shape,
// element type and memory space from its result type; copy's maps and
// operand segments from its bracketed index expressions), so printing a
// parsed module reproduces the text it came from.
#include "parse.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <unordered_map>

#include "ops.h"

namespace fir {
namespace {

bool identStart(char c) { return std::isalpha((unsigned char)c) || c == '_'; }
bool identChar(char c) {
  return std::isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$' || c == '-';
}

// Float value of a bit pattern of format `k` (the inverse of floatBits).
double floatFromBits(FloatKind k, uint64_t b) {
  switch (k) {
    case FloatKind::F64: {
      double d;
      std::memcpy(&d, &b, 8);
      return d;
    }
    case FloatKind::F32: {
      uint32_t u = (uint32_t)b;
      float f;
      std::memcpy(&f, &u, 4);
      return f;
    }
    case FloatKind::BF16: {
      uint32_t u = (uint32_t)(b & 0xffff) << 16;
      float f;
      std::memcpy(&f, &u, 4);
      return f;
    }
    default: break;
  }
  // Narrow IEEE-style formats: sign, exponent, mantissa.
  int mant = 10, ebits = 5;
  bool hasInf = true;
  if (k == FloatKind::E4M3FN) mant = 3, ebits = 4, hasInf = false;
  if (k == FloatKind::E5M2) mant = 2, ebits = 5;
  const int bias = (1 << (ebits - 1)) - 1;
  const uint64_t m = b & ((1ull << mant) - 1), e = (b >> mant) & ((1ull << ebits) - 1);
  const bool neg = (b >> (mant + ebits)) & 1;
  double v;
  if (e == (1ull << ebits) - 1 && (hasInf || m == (1ull << mant) - 1)) {
    v = (hasInf && m == 0) ? INFINITY : NAN;
  } else if (e == 0) {
    v = std::ldexp((double)m, 1 - bias - mant);
  } else {
    v = std::ldexp(1.0 + (double)m / (double)(1ull << mant), (int)e - bias);
  }
  return neg ? -v : v;
}

class Parser {
 public:
  Parser(Context* ctx, const std::string& text) : ctx_(ctx), s_(text) {}

  Operation* module() {
    ws();
    std::unique_ptr<Operation> top;
    if (peekKw("module")) {
      top = operation();
    } else {
      // Bare top-level operations: wrap them in a module.
      top = makeOp(ctx_, "builtin.module", Location{}, {}, {}, {}, 1);
      Block* body = top->region(0).emplaceBlock();
      while (ws(), p_ < s_.size()) body->pushBack(operation());
    }
    ws();
    if (p_ != s_.size()) error("unexpected text after the module");
    if (!top->is("builtin.module")) error("expected a module");
    return ctx_->adopt(std::move(top));
  }

 private:
  // ---- lexing ---------------------------------------------------------------
  [[noreturn]] void error(const std::string& msg) const {
    size_t line = 1, col = 1;
    for (size_t i = 0; i < p_ && i < s_.size(); ++i) {
      if (s_[i] == '\n') ++line, col = 1;
      else ++col;
    }
    throw InvalidArgument(std::to_string(line) + ":" + std::to_string(col) + ": " + msg);
  }

  void ws() {
    for (;;) {
      while (p_ < s_.size() && std::isspace((unsigned char)s_[p_])) ++p_;
      if (p_ + 1 < s_.size() && s_[p_] == '/' && s_[p_ + 1] == '/') {
        while (p_ < s_.size() && s_[p_] != '\n') ++p_;
        continue;
      }
      return;
    }
  }
  bool peek(char c) {
    ws();
    return p_ < s_.size() && s_[p_] == c;
  }
  bool eat(char c) {
    if (!peek(c)) return false;
    ++p_;
    return true;
  }
  void expect(char c) {
    if (!eat(c)) error(std::string("expected '") + c + "'");
  }
  bool eatStr(const char* t) {
    ws();
    const size_t n = std::strlen(t);
    if (s_.compare(p_, n, t) != 0) return false;
    p_ += n;
    return true;
  }
  bool peekKw(const char* kw) {
    ws();
    const size_t n = std::strlen(kw);
    return s_.compare(p_, n, kw) == 0 && (p_ + n >= s_.size() || !identChar(s_[p_ + n]));
  }
  bool eatKw(const char* kw) {
    if (!peekKw(kw)) return false;
    p_ += std::strlen(kw);
    return true;
  }
  void expectKw(const char* kw) {
    if (!eatKw(kw)) error(std::string("expected '") + kw + "'");
  }
  std::string ident() {
    ws();
    if (p_ >= s_.size() || !identStart(s_[p_])) error("expected an identifier");
    size_t b = p_;
    while (p_ < s_.size() && identChar(s_[p_])) ++p_;
    return s_.substr(b, p_ - b);
  }
  std::string ssaName() {
    ws();
    if (p_ >= s_.size() || s_[p_] != '%') error("expected an SSA value name");
    size_t b = p_++;
    while (p_ < s_.size() && (std::isalnum((unsigned char)s_[p_]) || s_[p_] == '_' ||
                              s_[p_] == '$' || s_[p_] == '.'))
      ++p_;
    if (p_ == b + 1) error("empty SSA value name");
    return s_.substr(b, p_ - b);
  }
  std::string symbol() {
    ws();
    if (!eat('@')) error("expected '@symbol'");
    if (peek('"')) return stringLit();
    size_t b = p_;
    while (p_ < s_.size() && identChar(s_[p_])) ++p_;
    return s_.substr(b, p_ - b);
  }
  int64_t integer() {
    ws();
    size_t b = p_;
    if (p_ < s_.size() && (s_[p_] == '-' || s_[p_] == '+')) ++p_;
    if (p_ >= s_.size() || !std::isdigit((unsigned char)s_[p_])) error("expected an integer");
    while (p_ < s_.size() && std::isdigit((unsigned char)s_[p_])) ++p_;
    return std::stoll(s_.substr(b, p_ - b));
  }
  std::string stringLit() {
    ws();
    if (!eat('"')) error("expected a string");
    std::string out;
    while (p_ < s_.size() && s_[p_] != '"') {
      char c = s_[p_++];
      if (c == '\\') {
        if (p_ >= s_.size()) break;
        char d = s_[p_];
        if (d == '"' || d == '\\') {
          out += d;
          ++p_;
        } else if (d == 'n') {
          out += '\n';
          ++p_;
        } else if (p_ + 1 < s_.size() && std::isxdigit((unsigned char)d) &&
                   std::isxdigit((unsigned char)s_[p_ + 1])) {
          out += (char)std::stoi(s_.substr(p_, 2), nullptr, 16);
          p_ += 2;
        } else {
          error("bad escape in string");
        }
      } else {
        out += c;
      }
    }
    if (!eat('"')) error("unterminated string");
    return out;
  }
  // A numeric literal: decimal integer / float, or 0x hex.  `isFloat` tells
  // whether it had a fraction or exponent; hex returns its bits.
  struct Number {
    std::string text;
    bool isFloat = false, isHex = false;
  };
  bool peekNumber() {
    ws();
    if (p_ >= s_.size()) return false;
    char c = s_[p_];
    if (std::isdigit((unsigned char)c)) return true;
    return (c == '-' || c == '+') && p_ + 1 < s_.size() && std::isdigit((unsigned char)s_[p_ + 1]);
  }
  Number number() {
    ws();
    Number n;
    size_t b = p_;
    if (s_.compare(p_, 2, "0x") == 0 || s_.compare(p_, 2, "0X") == 0) {
      p_ += 2;
      while (p_ < s_.size() && std::isxdigit((unsigned char)s_[p_])) ++p_;
      n.isHex = true;
      n.text = s_.substr(b, p_ - b);
      return n;
    }
    if (s_[p_] == '-' || s_[p_] == '+') ++p_;
    while (p_ < s_.size() && std::isdigit((unsigned char)s_[p_])) ++p_;
    if (p_ < s_.size() && s_[p_] == '.') {
      n.isFloat = true;
      ++p_;
      while (p_ < s_.size() && std::isdigit((unsigned char)s_[p_])) ++p_;
    }
    if (p_ < s_.size() && (s_[p_] == 'e' || s_[p_] == 'E')) {
      n.isFloat = true;
      ++p_;
      if (p_ < s_.size() && (s_[p_] == '-' || s_[p_] == '+')) ++p_;
      while (p_ < s_.size() && std::isdigit((unsigned char)s_[p_])) ++p_;
    }
    n.text = s_.substr(b, p_ - b);
    if (n.text.empty() || n.text == "-" || n.text == "+") error("expected a number");
    return n;
  }
  void skipLoc() {
    if (!eatKw("loc")) return;
    expect('(');
    int depth = 1;
    while (p_ < s_.size() && depth) {
      char c = s_[p_++];
      if (c == '"') {
        while (p_ < s_.size() && s_[p_] != '"') p_ += s_[p_] == '\\' ? 2 : 1;
        ++p_;
      } else if (c == '(') {
        ++depth;
      } else if (c == ')') {
        --depth;
      }
    }
  }

  // ---- types ------------------------------------------------------------------
  bool peekType() {
    ws();
    if (p_ >= s_.size()) return false;
    if (s_[p_] == '(') return true;
    static const char* kws[] = {"memref", "tensor", "index", "f16", "bf16", "f32", "f64",
                                "f8E4M3FN", "f8E5M2"};
    for (const char* k : kws)
      if (peekKw(k)) return true;
    if (s_[p_] == 'i' || (s_.compare(p_, 2, "si") == 0) || (s_.compare(p_, 2, "ui") == 0)) {
      size_t q = p_ + (s_[p_] == 'i' ? 1 : 2);
      size_t r = q;
      while (r < s_.size() && std::isdigit((unsigned char)s_[r])) ++r;
      return r > q && (r >= s_.size() || !identChar(s_[r]));
    }
    return false;
  }
  Type type() {
    ws();
    if (peek('(')) {  // function type
      expect('(');
      std::vector<Type> ins;
      if (!eat(')')) {
        do ins.push_back(type());
        while (eat(','));
        expect(')');
      }
      if (!eatStr("->")) error("expected '->' in a function type");
      std::vector<Type> outs;
      if (peek('(')) {
        expect('(');
        if (!eat(')')) {
          do outs.push_back(type());
          while (eat(','));
          expect(')');
        }
      } else {
        outs.push_back(type());
      }
      return ctx_->function(ins, outs);
    }
    if (eatKw("index")) return ctx_->index();
    if (eatKw("f16")) return ctx_->floatTy(FloatKind::F16);
    if (eatKw("bf16")) return ctx_->floatTy(FloatKind::BF16);
    if (eatKw("f32")) return ctx_->floatTy(FloatKind::F32);
    if (eatKw("f64")) return ctx_->floatTy(FloatKind::F64);
    if (eatKw("f8E4M3FN")) return ctx_->floatTy(FloatKind::E4M3FN);
    if (eatKw("f8E5M2")) return ctx_->floatTy(FloatKind::E5M2);
    if (eatKw("memref") || peekKw("tensor")) {
      const bool tensor = eatKw("tensor");
      expect('<');
      std::vector<int64_t> shape;
      Type elem;
      for (;;) {  // dims `NxMx...` then the element type
        ws();
        if (p_ < s_.size() && (std::isdigit((unsigned char)s_[p_]) || s_[p_] == '?')) {
          int64_t d = -1;
          if (s_[p_] == '?') ++p_;
          else d = integer();
          shape.push_back(d);
          if (p_ >= s_.size() || s_[p_] != 'x') error("expected 'x' in a shape");
          ++p_;
          continue;
        }
        elem = type();
        break;
      }
      if (tensor) {
        expect('>');
        return ctx_->tensor(shape, elem);
      }
      AffineMap layout;
      int64_t space = 0;
      while (eat(',')) {
        if (eatKw("affine_map")) {
          expect('<');
          layout = affineMapBody();
          expect('>');
        } else {
          space = integer();
        }
      }
      expect('>');
      return ctx_->memref(shape, elem, layout, space);
    }
    ws();
    Signedness sign = Signedness::Signless;
    if (s_.compare(p_, 2, "si") == 0) sign = Signedness::Signed, p_ += 2;
    else if (s_.compare(p_, 2, "ui") == 0) sign = Signedness::Unsigned, p_ += 2;
    else if (p_ < s_.size() && s_[p_] == 'i') ++p_;
    else error("expected a type");
    return ctx_->integer((unsigned)integer(), sign);
  }

  // ---- affine -------------------------------------------------------------------
  // Names of the map inputs: `d<i>` / `s<i>` in affine_map<...>, or SSA names
  // (and `symbol(%x)`) in a copy's bracketed index list.
  struct AffineScope {
    std::vector<std::string> dims, syms;
    bool ssa = false;                 // names are SSA values, collected as met
    std::vector<std::string> order;   // ssa: distinct names in order
  };
  AffineExpr affinePrimary(AffineScope& sc) {
    ws();
    if (eat('(')) {
      AffineExpr e = affineSum(sc);
      expect(')');
      return e;
    }
    if (eat('-')) return affinePrimary(sc) * (int64_t)-1;
    if (peekNumber()) return getAffineConstantExpr(integer(), ctx_);
    if (sc.ssa) {
      bool sym = eatKw("symbol");
      if (sym) expect('(');
      std::string n = ssaName();
      if (sym) expect(')');
      auto& list = sym ? sc.syms : sc.dims;
      for (unsigned i = 0; i < list.size(); ++i)
        if (list[i] == n) return sym ? getAffineSymbolExpr(i, ctx_) : getAffineDimExpr(i, ctx_);
      list.push_back(n);
      return sym ? getAffineSymbolExpr((unsigned)list.size() - 1, ctx_)
                 : getAffineDimExpr((unsigned)list.size() - 1, ctx_);
    }
    std::string n = ident();
    for (unsigned i = 0; i < sc.dims.size(); ++i)
      if (sc.dims[i] == n) return getAffineDimExpr(i, ctx_);
    for (unsigned i = 0; i < sc.syms.size(); ++i)
      if (sc.syms[i] == n) return getAffineSymbolExpr(i, ctx_);
    error("unknown affine identifier '" + n + "'");
  }
  AffineExpr affineProduct(AffineScope& sc) {
    AffineExpr e = affinePrimary(sc);
    for (;;) {
      if (eat('*')) e = e * affinePrimary(sc);
      else if (eatKw("floordiv")) e = floorDiv(e, affinePrimary(sc));
      else if (eatKw("ceildiv")) e = ceilDiv(e, affinePrimary(sc));
      else if (eatKw("mod")) e = e % affinePrimary(sc);
      else return e;
    }
  }
  AffineExpr affineSum(AffineScope& sc) {
    AffineExpr e = affineProduct(sc);
    for (;;) {
      ws();
      if (p_ + 1 < s_.size() && s_[p_] == '-' && s_[p_ + 1] == '>') return e;
      if (eat('+')) e = e + affineProduct(sc);
      else if (eat('-')) e = e - affineProduct(sc);
      else return e;
    }
  }
  // `(d0, d1)[s0] -> (e0, e1)`
  AffineMap affineMapBody() {
    AffineScope sc;
    expect('(');
    if (!eat(')')) {
      do sc.dims.push_back(ident());
      while (eat(','));
      expect(')');
    }
    if (eat('[')) {
      if (!eat(']')) {
        do sc.syms.push_back(ident());
        while (eat(','));
        expect(']');
      }
    }
    if (!eatStr("->")) error("expected '->' in an affine map");
    expect('(');
    std::vector<AffineExpr> res;
    if (!eat(')')) {
      do res.push_back(affineSum(sc));
      while (eat(','));
      expect(')');
    }
    return AffineMap::get((unsigned)sc.dims.size(), (unsigned)sc.syms.size(), res, ctx_);
  }

  // ---- attributes -----------------------------------------------------------------
  // A `#dialect.name<...>` attribute's text, brackets balanced.
  std::string hashAttrText() {
    ws();
    size_t b = p_;
    if (!eat('#')) error("expected '#'");
    while (p_ < s_.size() && identChar(s_[p_])) ++p_;
    ws();
    if (p_ < s_.size() && s_[p_] == '<') {
      int depth = 0;
      do {
        char c = s_[p_++];
        if (c == '"') {
          while (p_ < s_.size() && s_[p_] != '"') p_ += s_[p_] == '\\' ? 2 : 1;
          ++p_;
        } else if (c == '<' || c == '(' || c == '[' || c == '{') {
          ++depth;
        } else if (c == '>' || c == ')' || c == ']' || c == '}') {
          if (c == '>' && p_ >= 2 && s_[p_ - 2] == '-') continue;  // `->` inside
          --depth;
        }
      } while (p_ < s_.size() && depth > 0);
      if (depth) error("unbalanced attribute brackets");
    }
    return s_.substr(b, p_ - b);
  }

  double floatOf(const Number& n, FloatKind k) {
    if (n.isHex) return floatFromBits(k, std::stoull(n.text.substr(2), nullptr, 16));
    return std::strtod(n.text.c_str(), nullptr);
  }

  // dense<...> : tensor<...>
  Attribute dense() {
    expect('<');
    struct Elem {
      Number n;
      bool boolean = false, b = false;
    };
    std::vector<Elem> elems;
    std::function<void()> nested = [&]() {
      if (eat('[')) {
        if (!eat(']')) {
          do nested();
          while (eat(','));
          expect(']');
        }
        return;
      }
      Elem e;
      if (eatKw("true")) e.boolean = e.b = true;
      else if (eatKw("false")) e.boolean = true;
      else e.n = number();
      elems.push_back(e);
    };
    nested();
    expect('>');
    expect(':');
    Type t = type();
    if (!t.isTensor()) error("dense attribute needs a tensor type");
    Type el = t.elementType();
    if (el.isFloat()) {
      std::vector<double> v;
      for (auto& e : elems) v.push_back(floatOf(e.n, el.impl()->fkind));
      return Attribute::denseFloat(t, v);
    }
    std::vector<int64_t> v;
    for (auto& e : elems)
      v.push_back(e.boolean ? (int64_t)e.b
                            : e.n.isHex ? (int64_t)std::stoull(e.n.text.substr(2), nullptr, 16)
                                        : std::stoll(e.n.text));
    return Attribute::denseInt(t, v);
  }

  Attribute attribute() {
    ws();
    if (eatKw("true")) return Attribute::boolean(true);
    if (eatKw("false")) return Attribute::boolean(false);
    if (eatKw("unit")) return Attribute::unit();
    if (peek('"')) return Attribute::string(stringLit());
    if (eatKw("array")) {
      expect('<');
      if (!eatKw("i64")) error("only array<i64: ...> attributes are supported");
      std::vector<int64_t> v;
      if (eat(':')) {
        do v.push_back(integer());
        while (eat(','));
      }
      expect('>');
      return Attribute::denseI64(v);
    }
    if (eatKw("affine_map")) {
      expect('<');
      AffineMap m = affineMapBody();
      expect('>');
      return Attribute::affineMap(m);
    }
    if (eatKw("dense")) return dense();
    if (peek('#')) {
      size_t save = p_;
      std::string t = hashAttrText();
      auto inner = [&](const std::string& prefix) -> std::string {
        return t.compare(0, prefix.size(), prefix) == 0 && t.back() == '>'
                   ? t.substr(prefix.size(), t.size() - prefix.size() - 1)
                   : std::string();
      };
      std::string ms = inner("#frisk.memory_space<"), gp = inner("#frisk.gemm_warp_policy<");
      if (!ms.empty()) {
        if (ms == "Local") return Attribute::memorySpace(MemorySpace::Local);
        if (ms == "Global") return Attribute::memorySpace(MemorySpace::Global);
        if (ms == "Shared") return Attribute::memorySpace(MemorySpace::Shared);
        p_ = save;
        error("unknown memory space '" + ms + "'");
      }
      if (!gp.empty()) {
        static const char* names[] = {"Square", "FullRow", "FullCol", "Auto"};
        for (int i = 0; i < 4; ++i)
          if (gp == names[i]) return Attribute::gemmPolicy((GemmWarpPolicy)i);
        p_ = save;
        error("unknown gemm warp policy '" + gp + "'");
      }
      return Attribute::opaque(t);
    }
    if (peekNumber() || (p_ + 1 < s_.size() && s_[p_] == '0' && (s_[p_ + 1] == 'x'))) {
      Number n = number();
      Type t;
      if (eat(':')) t = type();
      if (!t) t = n.isFloat ? ctx_->floatTy(FloatKind::F64) : ctx_->integer(64);
      if (t.isFloat()) return Attribute::floating(t, floatOf(n, t.impl()->fkind));
      if (n.isFloat) error("float literal with a non-float type");
      return Attribute::integer(t, n.isHex ? (int64_t)std::stoull(n.text.substr(2), nullptr, 16)
                                           : std::stoll(n.text));
    }
    if (peekType()) return Attribute::typeAttr(type());
    error("expected an attribute");
  }

  // Before a region, `{` opens an attribute dictionary only when it holds
  // `name =`, `name,` or `name}` entries, or is `{}` followed by the region.
  bool peekAttrDict() {
    if (!peek('{')) return false;
    const size_t save = p_;
    ++p_;
    bool dict = false;
    if (eat('}')) {
      dict = peek('{');
    } else {
      ws();
      if (p_ < s_.size() && (identStart(s_[p_]) || s_[p_] == '"')) {
        if (s_[p_] == '"') stringLit();
        else while (p_ < s_.size() && identChar(s_[p_])) ++p_;
        dict = peek('=') || peek(',') || peek('}');
      }
    }
    p_ = save;
    return dict;
  }

  std::vector<NamedAttr> attrDict() {
    std::vector<NamedAttr> out;
    if (!eat('{')) return out;
    if (eat('}')) return out;
    do {
      ws();
      std::string name = peek('"') ? stringLit() : ident();
      Attribute v = eat('=') ? attribute() : Attribute::unit();
      out.push_back({name, v});
    } while (eat(','));
    expect('}');
    return out;
  }

  // ---- values -------------------------------------------------------------------------
  Value use(const std::string& n) {
    auto it = values_.find(n);
    if (it == values_.end()) {
      p_ -= n.size();  // report at the name (it was just read)
      error("use of undefined value " + n);
    }
    return it->second;
  }
  void define(const std::string& n, Value v) {
    if (values_.count(n)) error("redefinition of " + n);
    values_[n] = v;
  }
  std::vector<Value> operandList() {
    std::vector<Value> vs;
    if (!peek('%')) return vs;
    do vs.push_back(use(ssaName()));
    while (eat(','));
    return vs;
  }
  std::vector<Type> typeList() {
    std::vector<Type> ts;
    do ts.push_back(type());
    while (eat(','));
    return ts;
  }
  void checkTypes(const std::vector<Value>& vs, const std::vector<Type>& ts, const char* what) {
    if (vs.size() != ts.size()) error(std::string(what) + ": operand and type counts differ");
    for (size_t i = 0; i < vs.size(); ++i)
      if (vs[i].type() != ts[i])
        error(std::string(what) + ": operand " + std::to_string(i) + " has type " +
              vs[i].type().str() + ", not " + ts[i].str());
  }

  // ---- regions ------------------------------------------------------------------------
  // `{ [^bb0(args):] ops ... }`.  `entry` holds values already created as the
  // entry block's arguments (parallel ivs, function arguments) or is null.
  // `isolated` regions (function and kernel bodies) see no outer names and
  // keep theirs to themselves, as in MLIR.
  void region(Region& r, const std::vector<std::pair<std::string, Type>>* entryArgs,
              bool isolated = false) {
    std::unordered_map<std::string, Value> outer;
    if (isolated) outer.swap(values_);
    expect('{');
    Block* cur = r.emplaceBlock();
    if (entryArgs)
      for (auto& [n, t] : *entryArgs) {
        Value a = cur->addArgument(t);
        if (!n.empty()) define(n, a);
      }
    bool first = true;  // nothing parsed yet: a header names the entry block
    while (!peek('}')) {
      if (peek('^')) {
        ++p_;
        while (p_ < s_.size() && identChar(s_[p_])) ++p_;
        if (!first) cur = r.emplaceBlock();
        if (eat('(')) {
          if (!eat(')')) {
            do {
              std::string n = ssaName();
              expect(':');
              define(n, cur->addArgument(type()));
            } while (eat(','));
            expect(')');
          }
        }
        expect(':');
        first = false;
        continue;
      }
      cur->pushBack(operation());
      first = false;
    }
    expect('}');
    if (isolated) values_.swap(outer);
  }

  void ensureTerminator(Operation* op, const char* name) {
    for (auto& r : op->regions)
      for (auto& b : r->blocks)
        if (b->ops.empty() || !b->back()->is(name)) b->pushBack(makeOp(ctx_, name, op->loc, {}, {}));
  }

  // ---- operations ---------------------------------------------------------------------
  std::unique_ptr<Operation> operation() {
    ws();
    std::vector<std::string> results;
    std::vector<size_t> at;
    if (peek('%')) {
      do {
        ws();
        at.push_back(p_);
        results.push_back(ssaName());
      } while (eat(','));
      expect('=');
    }
    std::unique_ptr<Operation> op = opBody(results);
    skipLoc();
    if (op->numResults() != results.size()) {
      if (!at.empty()) p_ = at[0];
      error("'" + op->name + "' defines " + std::to_string(op->numResults()) + " results, " +
            std::to_string(results.size()) + " names given");
    }
    for (size_t i = 0; i < results.size(); ++i) {
      if (values_.count(results[i])) {
        p_ = at[i];
        error("redefinition of " + results[i]);
      }
      define(results[i], op->result((unsigned)i));
    }
    return op;
  }

  std::unique_ptr<Operation> make(const std::string& name, const std::vector<Value>& operands,
                                  const std::vector<Type>& results, std::vector<NamedAttr> attrs,
                                  unsigned regions = 0) {
    return makeOp(ctx_, name, Location{}, operands, results, std::move(attrs), regions);
  }

  std::unique_ptr<Operation> opBody(const std::vector<std::string>& results) {
    ws();
    if (peek('"')) return generic();
    if (eatKw("module")) {
      std::vector<NamedAttr> attrs;
      if (eatKw("attributes")) attrs = attrDict();
      auto op = make("builtin.module", {}, {}, attrs, 1);
      region(op->region(0), nullptr);
      return op;
    }
    if (eatKw("frisk.kernel")) {
      std::string name = symbol();
      expect('(');
      std::vector<Type> ins, outs;
      if (!eat(')')) {
        ins = typeList();
        expect(')');
      }
      if (eatStr("->")) {
        expect('(');
        if (!eat(')')) {
          outs = typeList();
          expect(')');
        }
      }
      Type fn = ctx_->function(ins, outs);
      auto op = make("frisk.kernel", {}, {},
                     {{"function_type", Attribute::typeAttr(fn)}, {"sym_name", Attribute::string(name)}},
                     1);
      region(op->region(0), nullptr, true);
      Block* entry = op->body();
      if (entry->numArguments() != ins.size())
        error("kernel @" + name + ": entry block arguments do not match its signature");
      for (auto& a : attrDict()) op->setAttr(a.name, a.value);
      return op;
    }
    if (eatKw("func.func")) {
      std::string name = symbol();
      expect('(');
      std::vector<std::pair<std::string, Type>> args;
      std::vector<Type> ins, outs;
      if (!eat(')')) {
        do {
          ws();
          std::string n;
          if (peek('%')) {
            n = ssaName();
            expect(':');
          }
          Type t = type();
          args.push_back({n, t});
          ins.push_back(t);
        } while (eat(','));
        expect(')');
      }
      if (eatStr("->")) {
        if (peek('(')) {
          expect('(');
          if (!eat(')')) {
            outs = typeList();
            expect(')');
          }
        } else {
          outs.push_back(type());
        }
      }
      auto op = make("func.func", {}, {},
                     {{"function_type", Attribute::typeAttr(ctx_->function(ins, outs))},
                      {"sym_name", Attribute::string(name)}},
                     1);
      if (eatKw("attributes"))
        for (auto& a : attrDict()) op->setAttr(a.name, a.value);
      if (peek('{')) region(op->region(0), &args, true);
      return op;
    }
    if (eatKw("frisk.parallel")) {
      auto ivs = ivList();
      expect('=');
      auto ranges = intTuple();
      expect(',');
      expectKw("threads");
      expect('=');
      int64_t threads = integer();
      auto op = make("frisk.parallel", {}, {},
                     {{"ranges", Attribute::denseI64(ranges)},
                      {"threads", Attribute::integer(ctx_->integer(64), threads)}},
                     1);
      region(op->region(0), &ivs);
      return op;
    }
    if (eatKw("frisk.block")) {
      auto ivs = ivList();
      expectKw("to");
      auto ranges = intTuple();
      auto op = make("frisk.block", {}, {}, {{"ranges", Attribute::denseI64(ranges)}}, 1);
      region(op->region(0), &ivs);
      ensureTerminator(op.get(), "frisk.end");
      return op;
    }
    if (eatKw("frisk.for")) {
      std::vector<std::pair<std::string, Type>> iv{{ssaName(), ctx_->index()}};
      expect('=');
      int64_t lo = integer();
      expectKw("to");
      int64_t hi = integer();
      int64_t step = 1;
      if (eatKw("step")) {
        expect('=');
        step = integer();
      }
      Type i64 = ctx_->integer(64);
      auto op = make("frisk.for", {}, {},
                     {{"lower", Attribute::integer(i64, lo)},
                      {"step", Attribute::integer(i64, step)},
                      {"upper", Attribute::integer(i64, hi)}},
                     1);
      region(op->region(0), &iv);
      ensureTerminator(op.get(), "frisk.end");
      return op;
    }
    if (eatKw("frisk.end")) return make("frisk.end", {}, {}, {});
    if (eatKw("frisk.gemm")) {
      expect('(');
      auto ops = operandList();
      expect(')');
      auto attrs = attrDict();
      expect(':');
      checkTypes(ops, typeList(), "frisk.gemm");
      return make("frisk.gemm", ops, {}, attrs);
    }
    if (eatKw("frisk.alloc_buffer")) {
      auto attrs = attrDict();
      if (!eatStr("->")) error("expected '->' after frisk.alloc_buffer");
      Type t = type();
      if (!t.isMemRef()) error("frisk.alloc_buffer produces a memref");
      auto op = make("frisk.alloc_buffer", {}, {t}, attrs);
      const int64_t sp = t.memorySpaceInt();
      op->setAttr("elementType", Attribute::typeAttr(t.elementType()));
      op->setAttr("memorySpace", Attribute::memorySpace((MemorySpace)sp));
      op->setAttr("shape", Attribute::denseI64(t.shape()));
      return op;
    }
    if (eatKw("frisk.copy")) {
      std::vector<Value> srcIdx, dstIdx;
      Value src = use(ssaName());
      AffineMap srcMap = bracketMap(srcIdx);
      expect(',');
      Value dst = use(ssaName());
      AffineMap dstMap = bracketMap(dstIdx);
      auto attrs = attrDict();
      expect(':');
      checkTypes({src, dst}, typeList(), "frisk.copy");
      std::vector<Value> operands{src, dst};
      operands.insert(operands.end(), srcIdx.begin(), srcIdx.end());
      operands.insert(operands.end(), dstIdx.begin(), dstIdx.end());
      auto op = make("frisk.copy", operands, {}, attrs);
      op->setAttr("srcMap", Attribute::affineMap(srcMap));
      op->setAttr("dstMap", Attribute::affineMap(dstMap));
      op->setAttr("operandSegmentSizes",
                  Attribute::denseI64({1, 1, (int64_t)srcIdx.size(), (int64_t)dstIdx.size()}));
      return op;
    }
    for (const char* n : {"frisk.fill", "frisk.reduce", "frisk.tile_store"}) {
      if (eatKw(n)) {
        auto ops = operandList();
        auto attrs = attrDict();
        expect(':');
        checkTypes(ops, typeList(), n);
        return make(n, ops, {}, attrs);
      }
    }
    if (eatKw("frisk.mma")) {
      auto ops = operandList();
      auto attrs = attrDict();
      expect(':');
      checkTypes(ops, typeList(), "frisk.mma");
      if (!eatStr("->")) error("expected '->' in frisk.mma");
      auto op = make("frisk.mma", ops, {type()}, attrs);
      // The assembly format elides these at their declared defaults.
      if (!op->hasAttr("trans_a")) op->setAttr("trans_a", Attribute::boolean(false));
      if (!op->hasAttr("trans_b")) op->setAttr("trans_b", Attribute::boolean(false));
      if (!op->hasAttr("policy")) op->setAttr("policy", Attribute::gemmPolicy(GemmWarpPolicy::Square));
      return op;
    }
    for (const char* n : {"frisk.reduce_tensor", "frisk.tile_load", "frisk.layout_view"}) {
      if (eatKw(n)) {
        auto ops = operandList();
        auto attrs = attrDict();
        expect(':');
        checkTypes(ops, typeList(), n);
        if (!eatStr("->")) error(std::string("expected '->' in ") + n);
        return make(n, ops, {type()}, attrs);
      }
    }
    if (eatKw("arith.constant")) {
      Attribute v = attribute();
      auto attrs = attrDict();
      Type t;
      switch (v.kind()) {
        case AttrKind::DenseFloat: case AttrKind::DenseInt: case AttrKind::Integer:
        case AttrKind::Float:
          t = v->type;
          break;
        case AttrKind::Bool: t = ctx_->integer(1); break;
        default: error("unsupported arith.constant value");
      }
      attrs.push_back({"value", v});
      return make("arith.constant", {}, {t}, attrs);
    }
    for (const char* n : {"arith.addf", "arith.maximumf", "arith.minimumf", "arith.mulf"}) {
      if (eatKw(n)) {
        auto ops = operandList();
        auto attrs = attrDict();
        expect(':');
        Type t = type();
        for (auto& v : ops)
          if (v.type() != t) error(std::string(n) + ": operand type differs from " + t.str());
        return make(n, ops, {t}, attrs);
      }
    }
    if (eatKw("memref.alloc")) {
      expect('(');
      auto ops = operandList();
      expect(')');
      auto attrs = attrDict();
      expect(':');
      return make("memref.alloc", ops, {type()}, attrs);
    }
    if (eatKw("scf.for")) {
      std::string iv = ssaName();
      expect('=');
      Value lb = use(ssaName());
      expectKw("to");
      Value ub = use(ssaName());
      expectKw("step");
      Value st = use(ssaName());
      std::vector<std::pair<std::string, Type>> args{{iv, lb.type()}};
      std::vector<Value> operands{lb, ub, st};
      std::vector<Type> resultTypes;
      if (eatKw("iter_args")) {
        expect('(');
        std::vector<std::string> names;
        do {
          names.push_back(ssaName());
          expect('=');
          operands.push_back(use(ssaName()));
        } while (eat(','));
        expect(')');
        if (!eatStr("->")) error("expected '->' after iter_args");
        expect('(');
        resultTypes = typeList();
        expect(')');
        if (resultTypes.size() != names.size()) error("scf.for: iter_args and result counts differ");
        for (size_t i = 0; i < names.size(); ++i) args.push_back({names[i], resultTypes[i]});
      }
      std::vector<NamedAttr> attrs;
      if (peekAttrDict()) attrs = attrDict();
      auto op = make("scf.for", operands, resultTypes, attrs, 1);
      region(op->region(0), &args);
      if (resultTypes.empty()) ensureTerminator(op.get(), "scf.yield");
      return op;
    }
    if (eatKw("scf.yield") || peekKw("return")) {
      const bool ret = eatKw("return");
      auto ops = operandList();
      if (!ops.empty()) {
        expect(':');
        checkTypes(ops, typeList(), ret ? "return" : "scf.yield");
      }
      auto attrs = attrDict();
      return make(ret ? "func.return" : "scf.yield", ops, {}, attrs);
    }
    (void)results;
    ws();
    const size_t at = p_;
    const std::string name = ident();
    p_ = at;
    error("unknown operation '" + name + "' (custom forms of this IR or \"generic\" form)");
  }

  std::vector<std::pair<std::string, Type>> ivList() {
    std::vector<std::pair<std::string, Type>> ivs;
    expect('(');
    if (!eat(')')) {
      do ivs.push_back({ssaName(), ctx_->index()});
      while (eat(','));
      expect(')');
    }
    return ivs;
  }
  std::vector<int64_t> intTuple() {
    std::vector<int64_t> v;
    expect('(');
    if (!eat(')')) {
      do v.push_back(integer());
      while (eat(','));
      expect(')');
    }
    return v;
  }
  // `[e0, e1]` over SSA names: the map and its index operands.
  AffineMap bracketMap(std::vector<Value>& idx) {
    expect('[');
    AffineScope sc;
    sc.ssa = true;
    std::vector<AffineExpr> res;
    if (!eat(']')) {
      do res.push_back(affineSum(sc));
      while (eat(','));
      expect(']');
    }
    if (res.empty()) return AffineMap::get(ctx_);
    for (auto& n : sc.dims) idx.push_back(use(n));
    for (auto& n : sc.syms) idx.push_back(use(n));
    return AffineMap::get((unsigned)sc.dims.size(), (unsigned)sc.syms.size(), res, ctx_);
  }

  // `"name"(%a, %b) [({...}, {...})] [{attrs}] : (types) -> (types)`
  std::unique_ptr<Operation> generic() {
    std::string name = stringLit();
    expect('(');
    auto ops = operandList();
    expect(')');
    std::vector<std::unique_ptr<Region>> regions;
    size_t save = p_;
    if (eat('(') && peek('{')) {
      do {
        regions.push_back(std::make_unique<Region>());
        region(*regions.back(), nullptr);
      } while (eat(','));
      expect(')');
    } else {
      p_ = save;
    }
    auto attrs = attrDict();
    expect(':');
    auto fn = type();
    if (!fn.isFunction()) error("generic operation needs a function type");
    checkTypes(ops, fn.inputs(), name.c_str());
    auto op = make(name, ops, fn.results(), attrs, 0);
    for (auto& r : regions) {
      Region* nr = op->addRegion();
      nr->takeBody(*r);
    }
    return op;
  }

  Context* ctx_;
  const std::string& s_;
  size_t p_ = 0;
  std::unordered_map<std::string, Value> values_;
};

}  // namespace

Operation* parseModule(Context* ctx, const std::string& text) {
  Parser p(ctx, text);
  return p.module();
}

}  // namespace fir
