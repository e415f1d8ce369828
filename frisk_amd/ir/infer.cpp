// Layout inference, cost model and execution export for CDNA4 (see infer.h).
#include "infer.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <numeric>
#include <set>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

namespace fir {

namespace {

bool isPow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int log2i(int64_t x) {
  int b = 0;
  while ((int64_t(1) << b) < x) ++b;
  return b;
}

// Rank over GF(2) of a set of bit vectors.
int gf2RankOf(std::vector<uint64_t> v) {
  int r = 0;
  for (int bit = 0; bit < 64 && r < (int)v.size(); ++bit) {
    auto it = std::find_if(v.begin() + r, v.end(), [&](uint64_t c) { return (c >> bit) & 1; });
    if (it == v.end()) continue;
    std::swap(*it, v[r]);
    for (size_t j = 0; j < v.size(); ++j)
      if ((int)j != r && ((v[j] >> bit) & 1)) v[j] ^= v[r];
    ++r;
  }
  return r;
}

std::string joinPairs(const std::vector<std::array<int64_t, 2>>& b, size_t from, size_t to) {
  std::ostringstream os;
  os << '[';
  for (size_t i = from; i < to; ++i) os << (i > from ? ", " : "") << '[' << b[i][0] << ", " << b[i][1] << ']';
  os << ']';
  return os.str();
}

const char* policyName(GemmWarpPolicy p) {
  switch (p) {
    case GemmWarpPolicy::Square: return "Square";
    case GemmWarpPolicy::FullRow: return "FullRow";
    case GemmWarpPolicy::FullCol: return "FullCol";
    case GemmWarpPolicy::Auto: return "Auto";
  }
  return "?";
}

// Input-kind throughput of one SIMD, multiply-adds counted as 2 flops
// (MI355X dense peaks / (1024 SIMDs x 2.4 GHz): 1024 flops/clk for
// bf16/f16, 2048 for fp8/i8, 64 for f32).
int64_t flopsPerClock(MfmaInput k) {
  switch (k) {
    case MfmaInput::F16: case MfmaInput::BF16: return 1024;
    case MfmaInput::FP8: case MfmaInput::I8: return 2048;
    case MfmaInput::F32: return 64;
  }
  return 1024;
}

int64_t elemBytes(Type t) { return std::max<int64_t>(1, t.bitWidth() / 8); }

}  // namespace

// ============================================================================
// Distributed layouts
// ============================================================================
std::array<int64_t, 2> DistLayout::at(uint64_t c) const {
  int64_t r = 0, col = 0;
  for (size_t i = 0; i < basis.size(); ++i)
    if ((c >> i) & 1) {
      r ^= basis[i][0];
      col ^= basis[i][1];
    }
  return {r, col};
}

int DistLayout::gf2Rank() const {
  const int rb = log2i(rows);
  std::vector<uint64_t> v;
  for (auto& b : basis) v.push_back((uint64_t)b[0] | ((uint64_t)b[1] << rb));
  return gf2RankOf(v);
}

bool DistLayout::coversTile() const { return gf2Rank() == log2i(rows) + log2i(cols); }

int64_t DistLayout::replication() const { return int64_t(1) << (carrierBits() - gf2Rank()); }

std::string DistLayout::str() const {
  std::ostringstream os;
  os << "#frisk.distributed<tile = [" << rows;
  if (rank == 2) os << ", " << cols;
  os << "], topology = [" << regs() << ", 64, " << waves() << "], reg = "
     << joinPairs(basis, 0, regBits) << ", lane = " << joinPairs(basis, regBits, regBits + 6)
     << ", wave = " << joinPairs(basis, regBits + 6, basis.size()) << ">";
  return os.str();
}

std::string distributedEncoding(const DistLayout& l) { return l.str(); }

DistLayout transposeLayout(const DistLayout& l) {
  DistLayout t = l;
  std::swap(t.rows, t.cols);
  for (auto& b : t.basis) std::swap(b[0], b[1]);
  return t;
}

std::optional<DistLayout> blockedLayout(int64_t rows, int64_t cols, int rank, int64_t threads,
                                        int64_t vec) {
  if (!isPow2(rows) || !isPow2(cols) || !isPow2(threads) || threads < 64 || !isPow2(vec) ||
      vec > cols)
    return std::nullopt;
  const int colBits = log2i(cols), linBits = log2i(rows) + colBits;
  const int vb = log2i(vec), wb = log2i(threads / 64);
  DistLayout l;
  l.rows = rows;
  l.cols = cols;
  l.rank = rank;
  l.waveBits = wb;
  l.regBits = std::max(vb, linBits - 6 - wb);
  l.basis.assign(l.carrierBits(), {0, 0});
  auto lin = [&](int j) -> std::array<int64_t, 2> {
    if (j >= linBits) return {0, 0};
    if (j < colBits) return {0, int64_t(1) << j};
    return {int64_t(1) << (j - colBits), 0};
  };
  int j = 0;
  for (int i = 0; i < vb; ++i) l.basis[i] = lin(j++);
  for (int i = 0; i < 6; ++i) l.basis[l.regBits + i] = lin(j++);
  for (int i = 0; i < wb; ++i) l.basis[l.regBits + 6 + i] = lin(j++);
  for (int i = vb; i < l.regBits; ++i) l.basis[i] = lin(j++);
  return l;
}

DistLayout sliceLayout(const DistLayout& l, int axis) {
  DistLayout s = l;
  s.rank = 1;
  s.rows = axis == 1 ? l.rows : l.cols;
  s.cols = 1;
  for (size_t i = 0; i < l.basis.size(); ++i) s.basis[i] = {axis == 1 ? l.basis[i][0] : l.basis[i][1], 0};
  return s;
}

bool equalUpToAxisPermutation(const DistLayout& a, const DistLayout& r, int axis,
                              std::vector<int64_t>* perm) {
  if (a.rows != r.rows || a.cols != r.cols || a.regBits != r.regBits || a.waveBits != r.waveBits)
    return false;
  const int other = 1 - axis;
  const int bits = log2i(axis == 0 ? a.rows : a.cols);
  // Pairs (required component x, actual component y); pi(x) = y must be a
  // well-defined linear bijection of the axis index space.
  std::vector<std::pair<uint64_t, uint64_t>> rowsXY;
  for (size_t i = 0; i < a.basis.size(); ++i) {
    if (a.basis[i][other] != r.basis[i][other]) return false;
    uint64_t x = (uint64_t)r.basis[i][axis], y = (uint64_t)a.basis[i][axis];
    // Reduce x against the current echelon, carrying y along.
    for (auto& p : rowsXY) {
      const int lead = 63 - __builtin_clzll(p.first);
      if ((x >> lead) & 1) {
        x ^= p.first;
        y ^= p.second;
      }
    }
    if (x == 0) {
      if (y != 0) return false;  // inconsistent: pi(0) != 0
      continue;
    }
    rowsXY.push_back({x, y});
    std::sort(rowsXY.begin(), rowsXY.end(), [](auto& p, auto& q) { return p.first > q.first; });
  }
  if ((int)rowsXY.size() != bits) return false;
  std::vector<uint64_t> ys;
  for (auto& p : rowsXY) ys.push_back(p.second);
  if (gf2RankOf(ys) != bits) return false;
  if (perm) {
    perm->assign(bits, 0);
    for (int j = 0; j < bits; ++j) {
      uint64_t x = uint64_t(1) << j, y = 0;
      for (auto& p : rowsXY) {
        const int lead = 63 - __builtin_clzll(p.first);
        if ((x >> lead) & 1) {
          x ^= p.first;
          y ^= p.second;
        }
      }
      (*perm)[j] = (int64_t)y;
    }
  }
  return true;
}

// ============================================================================
// MFMA bindings
// ============================================================================
namespace {

DistLayout fromGf2(const Gf2Map& m, int64_t rows, int64_t cols, int regBits, int waveBits) {
  DistLayout l;
  l.rows = rows;
  l.cols = cols;
  l.regBits = regBits;
  l.waveBits = waveBits;
  const int rb = log2i(rows);
  for (uint64_t c : m.cols)
    l.basis.push_back({(int64_t)(c & ((uint64_t(1) << rb) - 1)), (int64_t)(c >> rb)});
  return l;
}

std::optional<MmaGeometry> geometryWithAtom(int64_t m, int64_t n, int64_t k, const MfmaInstr& atom,
                                            int64_t threads, GemmWarpPolicy policy) {
  const int64_t waves = threads / 64;
  std::optional<MmaGeometry> best;
  int64_t bestScore = 0;
  for (int64_t gM = 1; gM <= waves; gM *= 2) {
    const int64_t gN = waves / gM;
    if (m % gM || n % gN) continue;
    const int64_t wm = m / gM, wn = n / gN;
    if (wm % atom.m || wn % atom.n || k % atom.k) continue;
    int64_t score = std::llabs(wm - wn);
    if (policy == GemmWarpPolicy::FullRow) score = -gM;
    if (policy == GemmWarpPolicy::FullCol) score = -gN;
    if (!best || score < bestScore) {
      best = MmaGeometry{m, n, k, threads, gM, gN, atom, wm / atom.m, wn / atom.n, k / atom.k};
      bestScore = score;
    }
  }
  return best;
}

std::optional<DistLayout> hwOperand(const MmaGeometry& g, char which) {
  auto map = cdna4FragmentGf2(g, which);
  if (!map) return std::nullopt;
  const int64_t regs = which == 'A' ? g.aRegs() : which == 'B' ? g.bRegs() : g.cRegs();
  const int64_t rows = which == 'B' ? g.k : g.m;
  const int64_t cols = which == 'A' ? g.k : g.n;
  return fromGf2(*map, rows, cols, log2i(regs), log2i(g.waves()));
}

}  // namespace

DistLayout MmaBinding::operand(char which) const {
  // Not swapped: A, B, C are the hardware fragments.  Swapped: the MFMAs
  // compute D^T = B'^T A'^T, so A' = (hw B)^T, B' = (hw A)^T, D = (hw C)^T.
  if (!swapped) return *hwOperand(hw, which);
  if (which == 'A') return transposeLayout(*hwOperand(hw, 'B'));
  if (which == 'B') return transposeLayout(*hwOperand(hw, 'A'));
  return transposeLayout(*hwOperand(hw, 'C'));
}

std::string MmaBinding::str() const {
  std::ostringstream os;
  os << "{atom = \"" << hw.atom.name << "\", wave_grid = [" << hw.gM << ", " << hw.gN
     << "], repeats = [" << hw.mRepeat << ", " << hw.nRepeat << ", " << hw.kRepeat
     << "], policy = \"" << policyName(policy) << "\", swapped = " << (swapped ? "true" : "false")
     << "}";
  return os.str();
}

std::vector<MmaBinding> cdna4MmaBindings(int64_t m, int64_t n, int64_t k, Type in, Type acc,
                                         int64_t threads, GemmWarpPolicy policy) {
  std::vector<MmaBinding> out;
  auto kind = mfmaInputOf(in);
  if (!kind || threads < 64 || threads > 1024 || !isPow2(threads)) return out;
  const bool accOk = *kind == MfmaInput::I8 ? acc.isSignlessInteger(32) : acc.isF32();
  if (!accOk) return out;
  for (bool swapped : {false, true}) {
    const int64_t hm = swapped ? n : m, hn = swapped ? m : n;
    for (const MfmaInstr& atom : cdna4MfmaTable()) {
      if (atom.input != *kind) continue;
      for (GemmWarpPolicy p : {GemmWarpPolicy::Square, GemmWarpPolicy::FullRow, GemmWarpPolicy::FullCol}) {
        auto g = geometryWithAtom(hm, hn, k, atom, threads, p);
        if (!g || !cdna4FragmentGf2(*g, 'A') || !cdna4FragmentGf2(*g, 'B') ||
            !cdna4FragmentGf2(*g, 'C'))
          continue;
        bool dup = false;
        for (auto& b : out)
          dup |= b.swapped == swapped && std::string(b.hw.atom.name) == atom.name &&
                 b.hw.gM == g->gM && b.hw.gN == g->gN;
        if (!dup) out.push_back(MmaBinding{*g, p, swapped});
      }
    }
  }
  if (policy != GemmWarpPolicy::Auto) {
    // Keep the bindings whose logical wave grid (the hardware grid, turned
    // around when the operands are swapped) is the policy's grid for that
    // atom on the logical (m, n).
    std::vector<MmaBinding> kept;
    for (const MmaBinding& b : out) {
      auto want = geometryWithAtom(m, n, k, b.hw.atom, threads, policy);
      const int64_t lm = b.swapped ? b.hw.gN : b.hw.gM, ln = b.swapped ? b.hw.gM : b.hw.gN;
      if (want && want->gM == lm && want->gN == ln) kept.push_back(b);
    }
    out = std::move(kept);
  }
  return out;
}

// ============================================================================
// Cost profile
// ============================================================================
const std::vector<std::string>& CostProfile::featureNames() {
  static const std::vector<std::string> names = {
      "mfma_cycles",         // MFMA issue cycles per wave
      "lds_read_cycles",     // LDS read cycles per workgroup (phases x conflict)
      "lds_read_issues",     // MMA fragment LDS read instructions per wave
      "lds_write_cycles",    // LDS write cycles per workgroup
      "global_lines",        // 128-byte lines touched per workgroup
      "valu_issues",         // VALU instructions per wave
      "trans_issues",        // transcendental VALU instructions per wave
      "reduction_shuffles",  // cross-lane exchange instructions per wave
      "conversion_bytes",    // bytes moved through LDS by layout conversions
      "barriers"};           // workgroup barriers
  return names;
}

const std::vector<std::string>& CostProfile::perWaveFeatures() {
  static const std::vector<std::string> names = {"mfma_cycles", "lds_read_issues", "valu_issues",
                                                 "trans_issues", "reduction_shuffles"};
  return names;
}

CostProfile CostProfile::defaults() {
  // Cycles per unit on MI355X.  MFMA cycles count 1:1.  LDS cycles are
  // modelled phases (16 lanes x 16 B at 64 banks of 4 B).  A 128-byte global
  // line takes 2 cycles of the 64 B/clk L1 return path.  A wave64 VALU op
  // issues over 4 cycles; transcendentals run at quarter rate (16).  A
  // cross-lane step is a DPP/permlane move plus the combine (8).  A fragment
  // LDS read instruction takes a wave64 issue slot (4): the transposing
  // 8-byte reads of M/N-major operands need twice the instructions of
  // ds_read_b128 for the same bytes, so the wave that reads more of the
  // transposed operand issues more.  LDS moves
  // 128 B/clk.  A workgroup barrier costs ~150 cycles (measured: the ping-pong
  // GEMM's extra barrier per phase cost 150 cycles, SQ_BUSY_CYCLES).
  CostProfile p;
  p.weights = {{"mfma_cycles", 1.0},       {"lds_read_cycles", 1.0},  {"lds_read_issues", 4.0},
               {"lds_write_cycles", 1.0},  {"global_lines", 2.0},     {"valu_issues", 4.0},
               {"trans_issues", 16.0},
               {"reduction_shuffles", 8.0}, {"conversion_bytes", 1.0 / 128.0}, {"barriers", 150.0}};
  return p;
}

namespace {
// Minimal JSON reader for {"id": "...", "weights": {"name": number, ...}}.
struct JsonCursor {
  const std::string& s;
  size_t i = 0;
  void ws() {
    while (i < s.size() && isspace((unsigned char)s[i])) ++i;
  }
  bool eat(char c) {
    ws();
    if (i < s.size() && s[i] == c) {
      ++i;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) throw InvalidArgument(std::string("cost-profile: expected '") + c + "'");
  }
  std::string str() {
    ws();
    expect('"');
    std::string out;
    while (i < s.size() && s[i] != '"') out += s[i++];
    expect('"');
    return out;
  }
  double num() {
    ws();
    size_t end = i;
    while (end < s.size() && (isdigit((unsigned char)s[end]) || strchr("+-.eE", s[end]))) ++end;
    if (end == i) throw InvalidArgument("cost-profile: expected a number");
    double v = std::stod(s.substr(i, end - i));
    i = end;
    return v;
  }
  bool boolean() {
    ws();
    for (const char* w : {"true", "false"})
      if (s.compare(i, strlen(w), w) == 0) {
        i += strlen(w);
        return w[0] == 't';
      }
    throw InvalidArgument("cost-profile: expected true or false");
  }
  // Reads past one value of any kind (provenance records).
  void skip() {
    ws();
    if (i >= s.size()) throw InvalidArgument("cost-profile: truncated");
    if (s[i] == '"') {
      str();
    } else if (s[i] == '{' || s[i] == '[') {
      const char close = s[i] == '{' ? '}' : ']';
      ++i;
      if (eat(close)) return;
      do {
        if (close == '}') {
          str();
          expect(':');
        }
        skip();
      } while (eat(','));
      expect(close);
    } else if (s[i] == 't' || s[i] == 'f') {
      boolean();
    } else if (s.compare(i, 4, "null") == 0) {
      i += 4;
    } else {
      num();
    }
  }
};
}  // namespace

CostProfile CostProfile::fromJson(const std::string& text) {
  CostProfile p = defaults();
  JsonCursor c{text};
  c.expect('{');
  if (c.eat('}')) return p;
  do {
    const std::string key = c.str();
    c.expect(':');
    if (key == "id") {
      p.id = c.str();
    } else if (key == "weights") {
      c.expect('{');
      if (!c.eat('}')) {
        do {
          const std::string f = c.str();
          c.expect(':');
          const double v = c.num();
          const auto& names = featureNames();
          if (std::find(names.begin(), names.end(), f) == names.end())
            throw InvalidArgument("cost-profile: unknown feature '" + f + "'");
          if (!(v >= 0) || !std::isfinite(v))
            throw InvalidArgument("cost-profile: weight of '" + f + "' must be finite and >= 0");
          p.weights[f] = v;
        } while (c.eat(','));
        c.expect('}');
      }
    } else if (key == "simd_share") {
      p.simdShare = c.boolean();
    } else if (key == "provenance") {
      c.skip();
    } else {
      throw InvalidArgument("cost-profile: unknown key '" + key + "'");
    }
  } while (c.eat(','));
  c.expect('}');
  return p;
}

// ============================================================================
// Inference
// ============================================================================
namespace {

using Features = std::map<std::string, double>;

// LDS access cost of one wave instruction: lanes' byte addresses, bytes per
// lane (4, 8 or 16).  Phases of 256 / bytes... lanes; a phase costs the
// largest number of distinct dwords in one of the 64 banks.
double ldsCycles(const std::vector<int64_t>& addrs, int64_t bytesPerLane) {
  const int64_t dw = std::max<int64_t>(1, bytesPerLane / 4);
  const int64_t lanesPerPhase = 64 / dw;
  double total = 0;
  for (size_t p = 0; p < addrs.size(); p += lanesPerPhase) {
    std::unordered_map<int64_t, std::vector<int64_t>> banks;
    for (size_t l = p; l < std::min(addrs.size(), p + lanesPerPhase); ++l)
      for (int64_t w = 0; w < dw; ++w) {
        const int64_t d = addrs[l] / 4 + w;
        auto& v = banks[((d % 64) + 64) % 64];
        if (std::find(v.begin(), v.end(), d) == v.end()) v.push_back(d);
      }
    size_t worst = 1;
    for (auto& kv : banks) worst = std::max(worst, kv.second.size());
    total += (double)worst;
  }
  return total;
}

struct UnionFind {
  std::vector<int> p;
  int add() {
    p.push_back((int)p.size());
    return (int)p.size() - 1;
  }
  int find(int x) { return p[x] == x ? x : p[x] = find(p[x]); }
  void unite(int a, int b) {
    a = find(a);
    b = find(b);
    if (a != b) p[std::max(a, b)] = std::min(a, b);
  }
};

struct StorageCand {
  std::optional<SwizzleProposal> swz;  // nullopt = row-major identity
  std::string str(int64_t rowBytes) const {
    std::ostringstream os;
    os << "#frisk.storage<space = \"lds\", row_bytes = " << rowBytes << ", swizzle = \""
       << (swz ? swz->formula : std::string("c")) << "\">";
    return os.str();
  }
  int64_t offset(int64_t rowBytes, int64_t row, int64_t byte) const {
    return swz ? swz->offset(row, byte) : row * rowBytes + byte;
  }
};

enum class VarKind { Mma, Storage, Free };

struct Var {
  VarKind kind;
  std::string name;
  int64_t domain = 0;
  int index = -1;  // mma / storage / class index
};

struct MmaSite {
  Operation* op;
  int64_t m, n, k, threads;
  bool ta, tb;
  Type in, acc;
  std::vector<MmaBinding> bindings;
  std::vector<std::array<DistLayout, 3>> layouts;  // per binding: A, B, C (over operand shapes)
  int var = -1;
};

struct StorageRoot {
  Value root;  // memref.alloc result in LDS
  int64_t rows = 1, rowBytes = 0, eb = 1;
  std::vector<StorageCand> cands;
  int var = -1;
};

struct ClassInfo {
  int64_t rows = 1, cols = 1;
  int rank = 2;
  Type elem;
  int64_t threads = 64;
  int mmaDef = -1;       // mma site whose result defines the class
  int reduceSrc = -1;    // class reduced into this one
  int reduceAxis = 0;
  int freeVar = -1;      // variable index when no contract defines it
  std::vector<DistLayout> freeCands;
  std::vector<Value> members;
};

class Inference {
 public:
  Inference(Operation* module, const InferOptions& o) : mod_(module), opts_(o) {}

  InferReport run() {
    rep_.costModelId = opts_.profile.id;
    try {
      collect();
      solve();
      if (rep_.status == "failed") return rep_;
      if (!opts_.analysisOnly) materialize();
    } catch (const InvalidArgument& e) {
      rep_.status = "failed";
      rep_.failure = e.what();
    }
    return rep_;
  }

 private:
  Operation* mod_;
  InferOptions opts_;
  InferReport rep_;
  UnionFind uf_;
  std::unordered_map<ValueImpl*, int> node_;
  std::vector<Value> nodeValue_;
  std::vector<MmaSite> mmas_;
  std::vector<StorageRoot> roots_;
  std::unordered_map<ValueImpl*, int> rootOf_;  // memref value -> root index
  std::vector<ClassInfo> classes_;
  std::unordered_map<int, int> classOfRoot_;    // uf root -> class index
  std::vector<Var> vars_;
  std::vector<Operation*> ops_;                 // ops inside parallel regions, in order
  std::unordered_map<Operation*, int64_t> threadsOf_;
  std::vector<int64_t> best_;
  // Solution-time state.
  std::vector<std::optional<DistLayout>> layouts_;
  // Memoized pure cost queries (keyed by the op, the layout and the storage
  // choice they depend on); reuse only, never changes a score.
  std::unordered_map<std::string, double> memo_;

  static std::string layoutKey(const DistLayout& l) {
    std::string k = std::to_string(l.rows) + "x" + std::to_string(l.cols) + ":" + std::to_string(l.regBits) +
                    ":" + std::to_string(l.waveBits);
    for (auto& b : l.basis) k += "," + std::to_string(b[0]) + "/" + std::to_string(b[1]);
    return k;
  }
  int64_t storageChoice(Value memref, const std::vector<int64_t>& asg) {
    const int ri = storageRootOf(rootMemref(memref));
    return ri < 0 ? -1 : ri * 1000 + asg[roots_[ri].var];
  }

  [[noreturn]] void fail(Operation* op, const std::string& what) {
    throw InvalidArgument("layout-inference: " + what + (op ? " (" + op->name + ")" : ""));
  }

  int nodeFor(Value v) {
    auto it = node_.find(v.impl());
    if (it != node_.end()) return it->second;
    const int id = uf_.add();
    node_[v.impl()] = id;
    nodeValue_.push_back(v);
    return id;
  }
  int classOf(Value v) {
    auto it = node_.find(v.impl());
    if (it == node_.end()) return -1;
    auto c = classOfRoot_.find(uf_.find(it->second));
    return c == classOfRoot_.end() ? -1 : c->second;
  }

  static bool isElementwise(const Operation* op) {
    const std::string& n = op->name;
    if (n.rfind("arith.", 0) == 0) return n != "arith.constant";
    return n.rfind("math.", 0) == 0;
  }
  static bool isTranscendental(const Operation* op) {
    return op->is("math.exp") || op->is("math.exp2") || op->is("math.log") ||
           op->is("math.rsqrt") || op->is("math.sqrt") || op->is("arith.divf");
  }

  Value rootMemref(Value v) {
    while (Operation* d = v.definingOp()) {
      if (d->is("frisk.layout_view") && d->numOperands() == 1) v = d->operand(0);
      else break;
    }
    return v;
  }
  int storageRootOf(Value memref) {
    auto it = rootOf_.find(memref.impl());
    return it == rootOf_.end() ? -1 : it->second;
  }

  // ---- collection -----------------------------------------------------------
  void collect() {
    Attribute t = mod_->attr("frisk.target");
    if (!t || t.kind() != AttrKind::String || t->s != "gfx950")
      fail(mod_, "cdna4-target: requires frisk.target = \"gfx950\"");
    mod_->walk([&](Operation* op) {
      if (op->is("frisk.gemm") || op->is("frisk.copy_legacy") || op->is("frisk.reduce"))
        fail(op, "input-verification: run frisk.normalize_layout_ir first");
    });
    // Ops inside parallel regions (or a kernel without one) with their
    // execution thread count.
    mod_->walk([&](Operation* op) {
      if (op->is("frisk.parallel")) {
        const int64_t th = op->intAttr("threads");
        op->region(0).walk([&](Operation* inner) { threadsOf_[inner] = th; });
      }
    });
    mod_->walk([&](Operation* op) {
      if (!threadsOf_.count(op)) {
        if (Attribute a = op->attr("frisk.execution_threads"); a && a.kind() == AttrKind::Integer)
          threadsOf_[op] = a->i;
      }
    });
    // Pre-order list in program order.
    std::function<void(Block*)> visit = [&](Block* b) {
      for (auto& o : b->ops) {
        ops_.push_back(o.get());
        for (auto& r : o->regions)
          for (auto& blk : r->blocks) visit(blk.get());
      }
    };
    for (auto& r : mod_->regions)
      for (auto& blk : r->blocks) visit(blk.get());

    // LDS storage roots.
    for (Operation* op : ops_) {
      if (op->is("memref.alloc") || op->is("frisk.alloc_buffer")) {
        Type mt = op->result(0).type();
        if (!mt.isMemRef() || mt.memorySpaceInt() != 3 || !mt.hasStaticShape()) continue;
        StorageRoot r;
        r.root = op->result(0);
        r.eb = elemBytes(mt.elementType());
        r.rows = mt.rank() >= 2 ? mt.numElements() / mt.dim(mt.rank() - 1) : 1;
        r.rowBytes = mt.dim(mt.rank() - 1) * r.eb;
        r.cands.push_back(StorageCand{});
        if (mt.rank() == 2 && isPow2(r.rowBytes) && r.rowBytes >= 32) {
          for (int atom : {32, 16}) {
            SwizzleProposal p = proposeLdsSwizzle(r.rowBytes, atom);
            bool dup = p.terms.empty();
            for (auto& c : r.cands)
              if (c.swz && c.swz->formula == p.formula) dup = true;
            if (!dup) r.cands.push_back(StorageCand{p});
          }
        }
        rootOf_[r.root.impl()] = (int)roots_.size();
        roots_.push_back(std::move(r));
      }
    }
    for (Operation* op : ops_)
      if (op->is("frisk.layout_view") && op->numOperands() == 1) {
        const int r = storageRootOf(rootMemref(op->operand(0)));
        if (r >= 0) rootOf_[op->result(0).impl()] = r;
      }

    // Tensor nodes and same-layout unions.
    for (Operation* op : ops_) {
      for (unsigned i = 0; i < op->numResults(); ++i)
        if (op->result(i).type().isTensor()) nodeFor(op->result(i));
      for (auto& r : op->regions)
        for (auto& blk : r->blocks)
          for (unsigned i = 0; i < blk->numArguments(); ++i)
            if (blk->argument(i).type().isTensor()) nodeFor(blk->argument(i));
    }
    for (Operation* op : ops_) {
      if (isElementwise(op)) {
        std::vector<Value> vs;
        for (Value v : op->operands)
          if (v.type().isTensor()) vs.push_back(v);
        for (unsigned i = 0; i < op->numResults(); ++i) vs.push_back(op->result(i));
        for (size_t i = 1; i < vs.size(); ++i)
          if (vs[i].type().shape() == vs[0].type().shape()) uf_.unite(nodeFor(vs[0]), nodeFor(vs[i]));
      } else if (op->is("frisk.mma")) {
        uf_.unite(nodeFor(op->operand(2)), nodeFor(op->result(0)));
      } else if (op->is("linalg.broadcast") && op->numOperands() == 2 && op->numResults() == 1) {
        uf_.unite(nodeFor(op->operand(1)), nodeFor(op->result(0)));
      } else if (op->is("frisk.convert_layout")) {
        fail(op, "input-verification: module already holds layout conversions");
      } else if (op->is("scf.for")) {
        Block* body = op->body();
        const unsigned nIter = op->numResults();
        const unsigned firstInit = op->numOperands() - nIter;
        Operation* yield = body ? body->terminator() : nullptr;
        for (unsigned i = 0; i < nIter; ++i) {
          if (!op->result(i).type().isTensor()) continue;
          const int r = nodeFor(op->result(i));
          uf_.unite(r, nodeFor(op->operand(firstInit + i)));
          if (body && body->numArguments() > i + 1) uf_.unite(r, nodeFor(body->argument(i + 1)));
          if (yield && yield->numOperands() > i) uf_.unite(r, nodeFor(yield->operand(i)));
        }
      }
    }
    // Classes.
    for (size_t i = 0; i < nodeValue_.size(); ++i) {
      const int root = uf_.find((int)i);
      auto it = classOfRoot_.find(root);
      int c;
      if (it == classOfRoot_.end()) {
        c = (int)classes_.size();
        classOfRoot_[root] = c;
        ClassInfo ci;
        Type t = nodeValue_[i].type();
        ci.rank = (int)t.rank();
        if (ci.rank < 1 || ci.rank > 2) fail(nodeValue_[i].definingOp(), "tensor-rank: only rank 1 and 2 tiles");
        ci.rows = t.dim(0);
        ci.cols = ci.rank == 2 ? t.dim(1) : 1;
        if (!isPow2(ci.rows) || !isPow2(ci.cols))
          fail(nodeValue_[i].definingOp(), "tensor-shape: extents must be powers of two");
        ci.elem = t.elementType();
        classes_.push_back(ci);
      } else {
        c = it->second;
      }
      classes_[c].members.push_back(nodeValue_[i]);
      Operation* d = nodeValue_[i].definingOp();
      Operation* owner = d ? d : nodeValue_[i].ownerBlock()->parentOp();
      if (owner && threadsOf_.count(owner)) classes_[c].threads = threadsOf_[owner];
    }
    // MMA sites.
    for (Operation* op : ops_) {
      if (!op->is("frisk.mma")) continue;
      MmaSite s;
      s.op = op;
      s.m = op->intAttr("m");
      s.n = op->intAttr("n");
      s.k = op->intAttr("k");
      s.ta = op->hasAttr("trans_a") && op->boolAttr("trans_a");
      s.tb = op->hasAttr("trans_b") && op->boolAttr("trans_b");
      s.in = op->operand(0).type().elementType();
      s.acc = op->result(0).type().elementType();
      s.threads = threadsOf_.count(op) ? threadsOf_[op] : 128;
      // frisk.mma's policy defaults to Square (FriskLayoutOps.td:42-43).
      const GemmWarpPolicy policy = op->hasAttr("policy") ? (GemmWarpPolicy)op->intAttr("policy")
                                                          : GemmWarpPolicy::Square;
      s.bindings = cdna4MmaBindings(s.m, s.n, s.k, s.in, s.acc, s.threads, policy);
      if (s.bindings.empty())
        fail(op, "instruction-contract: no MFMA binding for this shape, type and thread count");
      for (const MmaBinding& b : s.bindings)
        s.layouts.push_back({computeOperandLayout(s, b, 'A'), computeOperandLayout(s, b, 'B'),
                             computeOperandLayout(s, b, 'C')});
      const int c = classOf(op->result(0));
      if (classes_[c].mmaDef < 0) classes_[c].mmaDef = (int)mmas_.size();
      mmas_.push_back(s);
    }
    // Reductions define their result class from the source class.
    for (Operation* op : ops_) {
      if (!op->is("frisk.reduce_tensor")) continue;
      const int src = classOf(op->operand(0)), dst = classOf(op->result(0));
      ClassInfo& d = classes_[dst];
      if (d.mmaDef >= 0 || (d.reduceSrc >= 0 && (d.reduceSrc != src || d.reduceAxis != op->intAttr("dim"))))
        fail(op, "reduction-contract: result class has a conflicting definition");
      d.reduceSrc = src;
      d.reduceAxis = (int)op->intAttr("dim");
    }
    // Variables: MMA bindings, LDS storage, free classes.
    for (size_t i = 0; i < mmas_.size(); ++i) {
      mmas_[i].var = (int)vars_.size();
      vars_.push_back({VarKind::Mma, "mma#" + std::to_string(i), (int64_t)mmas_[i].bindings.size(), (int)i});
    }
    for (size_t i = 0; i < roots_.size(); ++i) {
      roots_[i].var = (int)vars_.size();
      vars_.push_back({VarKind::Storage, "lds#" + std::to_string(i), (int64_t)roots_[i].cands.size(), (int)i});
    }
    for (size_t c = 0; c < classes_.size(); ++c) {
      ClassInfo& ci = classes_[c];
      if (ci.mmaDef >= 0 || ci.reduceSrc >= 0) continue;
      // A class with no defining contract: operands of an MMA take that
      // binding's fragment (resolved at evaluation); otherwise blocked
      // layouts with 1..16 B per lane.
      bool mmaOperand = false;
      for (Value v : ci.members)
        for (Operation* u : v.users())
          if (u->is("frisk.mma") && (u->operand(0) == v || u->operand(1) == v)) mmaOperand = true;
      if (mmaOperand) continue;
      const int64_t eb = elemBytes(ci.elem);
      for (int64_t vec = 1; vec * eb <= 16 && vec <= ci.cols; vec *= 2)
        if (auto l = blockedLayout(ci.rows, ci.cols, ci.rank, ci.threads, vec)) ci.freeCands.push_back(*l);
      if (ci.freeCands.empty()) fail(ci.members[0].definingOp(), "candidate-generation: empty layout domain");
      ci.freeVar = (int)vars_.size();
      vars_.push_back({VarKind::Free, "value#" + std::to_string(c), (int64_t)ci.freeCands.size(), (int)c});
    }
    rep_.variables = (int64_t)vars_.size();
    // Graph listing.
    for (size_t i = 0; i < mmas_.size(); ++i)
      rep_.graph.push_back("hard instruction-contract mma#" + std::to_string(i) + " domain " +
                           std::to_string(mmas_[i].bindings.size()));
    for (size_t i = 0; i < roots_.size(); ++i)
      rep_.graph.push_back("storage lds#" + std::to_string(i) + " row_bytes " +
                           std::to_string(roots_[i].rowBytes) + " domain " +
                           std::to_string(roots_[i].cands.size()));
    for (size_t c = 0; c < classes_.size(); ++c) {
      const ClassInfo& ci = classes_[c];
      std::string d = ci.mmaDef >= 0 ? "defined by mma#" + std::to_string(ci.mmaDef)
                      : ci.reduceSrc >= 0 ? "reduction of value#" + std::to_string(ci.reduceSrc)
                      : ci.freeVar >= 0 ? "free, domain " + std::to_string(ci.freeCands.size())
                                        : "operand of an mma";
      rep_.graph.push_back("value#" + std::to_string(c) + " " + std::to_string(ci.rows) +
                           (ci.rank == 2 ? "x" + std::to_string(ci.cols) : "") + " (" +
                           std::to_string(ci.members.size()) + " SSA values) " + d);
    }
  }

  // ---- layouts under an assignment -----------------------------------------
  // Operand layout required by MMA site s (binding b) for 'A', 'B' or 'C',
  // expressed over the operand value's own shape (transposes applied).
  static DistLayout computeOperandLayout(const MmaSite& s, const MmaBinding& b, char which) {
    DistLayout l = b.operand(which);
    if ((which == 'A' && s.ta) || (which == 'B' && s.tb)) l = transposeLayout(l);
    return l;
  }
  const DistLayout& mmaOperandLayout(const MmaSite& s, const MmaBinding& b, char which) const {
    const size_t i = &b - s.bindings.data();
    return s.layouts[i][which == 'A' ? 0 : which == 'B' ? 1 : 2];
  }

  std::optional<DistLayout> classLayout(int c, const std::vector<int64_t>& asg) {
    if (layouts_[c]) return layouts_[c];
    ClassInfo& ci = classes_[c];
    std::optional<DistLayout> l;
    if (ci.mmaDef >= 0) {
      const MmaSite& s = mmas_[ci.mmaDef];
      if (asg[s.var] < 0) return std::nullopt;
      l = mmaOperandLayout(s, s.bindings[asg[s.var]], 'C');
    } else if (ci.reduceSrc >= 0) {
      auto src = classLayout(ci.reduceSrc, asg);
      if (!src) return std::nullopt;
      l = sliceLayout(*src, ci.reduceAxis);
    } else if (ci.freeVar >= 0) {
      if (asg[ci.freeVar] < 0) return std::nullopt;
      l = ci.freeCands[asg[ci.freeVar]];
    } else {
      // Operand-only class: the first consuming MMA's fragment.
      for (Value v : ci.members)
        for (Operation* u : v.users())
          if (u->is("frisk.mma")) {
            for (auto& s : mmas_)
              if (s.op == u) {
                if (asg[s.var] < 0) return std::nullopt;
                const char w = u->operand(0) == v ? 'A' : 'B';
                l = mmaOperandLayout(s, s.bindings[asg[s.var]], w);
                break;
              }
            if (l) break;
          }
    }
    layouts_[c] = l;
    return l;
  }

  // Byte address of logical element (r, c) of an LDS memref view.
  int64_t ldsAddress(Value memref, int64_t r, int64_t c, const std::vector<int64_t>& asg) {
    const int ri = storageRootOf(rootMemref(memref));
    Type t = memref.type();
    const int64_t eb = elemBytes(t.elementType());
    if (ri < 0) return (r * t.dim(t.rank() - 1) + c) * eb;
    const StorageRoot& root = roots_[ri];
    const StorageCand& cand = root.cands[std::max<int64_t>(0, asg[root.var])];
    return cand.offset(root.rowBytes, r, c * eb);
  }

  // ---- cost terms -----------------------------------------------------------
  // Each returns false when a layout it needs is not determined yet.
  bool costMma(const MmaSite& s, const std::vector<int64_t>& asg, Features& f, std::vector<std::string>* conv) {
    if (asg[s.var] < 0) return false;
    const MmaBinding& b = s.bindings[asg[s.var]];
    const MfmaInstr& a = b.hw.atom;
    f["mfma_cycles"] += (double)b.mfmaPerWave() * (2.0 * a.m * a.n * a.k / flopsPerClock(a.input));
    Operation* op = s.op;
    for (int w = 0; w < 2; ++w) {
      Value v = op->operand(w);
      const char which = w == 0 ? 'A' : 'B';
      const DistLayout& req = mmaOperandLayout(s, b, which);
      if (v.type().isMemRef()) {
        if (v.type().memorySpaceInt() != 3) continue;  // operands in global memory are not costed
        const int ri = storageRootOf(rootMemref(v));
        if (ri >= 0 && asg[roots_[ri].var] < 0) return false;
        const std::string key = "fr" + std::to_string((uintptr_t)op) + ":" + std::to_string(w) + ":" +
                                std::to_string(asg[s.var]) + ":" + std::to_string(storageChoice(v, asg));
        auto it = memo_.find(key);
        if (it == memo_.end()) {
          double issues = 0;
          const double cycles = fragmentReadCycles(v, req, which == 'A' ? !s.ta : s.tb, asg, issues);
          memo_.emplace(key + ":issues", issues);
          it = memo_.emplace(key, cycles).first;
        }
        f["lds_read_cycles"] += it->second;
        f["lds_read_issues"] += memo_.at(key + ":issues");
      } else {
        const int c = classOf(v);
        auto have = classLayout(c, asg);
        if (!have) return false;
        const Value other = op->operand(1 - w);
        bool ok = *have == req;
        // The k index may be permuted when the other operand is read from
        // memory with the same permutation.
        const int kAxis = (which == 'A') != (which == 'A' ? s.ta : s.tb) ? 1 : 0;
        if (!ok && other.type().isMemRef()) ok = equalUpToAxisPermutation(*have, req, kAxis);
        if (!ok) addConversion(op, w, v, f, conv);
      }
    }
    // Accumulator input: must hold the C fragment.
    Value init = op->operand(2);
    if (!init.definingOp() || !init.definingOp()->is("arith.constant")) {
      auto have = classLayout(classOf(init), asg);
      if (!have) return false;
      if (*have != mmaOperandLayout(s, b, 'C')) addConversion(op, 2, init, f, conv);
    }
    return true;
  }

  void addConversion(Operation* op, unsigned operand, Value v, Features& f, std::vector<std::string>* conv) {
    const int64_t bytes = v.type().numElements() * elemBytes(v.type().elementType());
    f["conversion_bytes"] += 2.0 * (double)bytes;
    f["barriers"] += 1.0;
    if (conv) conv->push_back(op->name + "#" + std::to_string(operand) + ": " + std::to_string(bytes) + " B");
  }

  // LDS cycles of reading an MMA operand fragment `l` (over the memref's own
  // shape) from `memref`; kContig: the per-lane k run is along the memref's
  // contiguous dimension.  `issues` receives the read instructions one wave
  // issues.
  double fragmentReadCycles(Value memref, const DistLayout& l, bool kContig, const std::vector<int64_t>& asg,
                            double& issues) {
    Type t = memref.type();
    const int64_t eb = elemBytes(t.elementType());
    // Per-lane vector: the consecutive register bits that walk the
    // contiguous (column) axis of the memref in order.
    int vb = 0;
    while (vb < l.regBits && l.basis[vb][0] == 0 && l.basis[vb][1] == (int64_t(1) << vb)) ++vb;
    int64_t vecElems = int64_t(1) << vb;
    int64_t bytes = std::min<int64_t>(16, vecElems * eb);
    vecElems = std::max<int64_t>(1, bytes / eb);
    if (!kContig && eb == 2) {
      // The k run is strided: gfx950's ds_read_b64_tr_b16 reads 8 B of a
      // row per lane and transposes inside 16-lane groups, delivering 4
      // k-consecutive elements per lane (modelled at the lanes' first element).
      vecElems = 4;
      bytes = 8;
    } else if (!kContig && eb == 1) {
      // ds_read_b64_tr_b8 likewise delivers 8 k-consecutive bytes per lane.
      vecElems = 8;
      bytes = 8;
    }
    double cycles = 0;
    const int64_t instrPerLane = std::max<int64_t>(1, l.regs() / vecElems);
    issues = (double)instrPerLane;
    for (int64_t wv = 0; wv < l.waves(); ++wv)
      for (int64_t ins = 0; ins < instrPerLane; ++ins) {
        std::vector<int64_t> addrs(64);
        for (int64_t lane = 0; lane < 64; ++lane) {
          auto rc = l.at(ins * vecElems, lane, wv);
          addrs[lane] = ldsAddress(memref, rc[0], rc[1], asg);
        }
        cycles += ldsCycles(addrs, std::max<int64_t>(4, bytes));
      }
    return cycles;
  }

  bool costReduce(Operation* op, const std::vector<int64_t>& asg, Features& f) {
    auto src = classLayout(classOf(op->operand(0)), asg);
    if (!src) return false;
    const int axis = (int)op->intAttr("dim");
    int inLane = 0, lanes = 0, waves = 0;
    for (int i = 0; i < src->carrierBits(); ++i) {
      const auto& b = src->basis[i];
      if (b[axis] == 0) continue;  // does not walk the reduced axis
      if (i < src->regBits) ++inLane;
      else if (i < src->regBits + 6) ++lanes;
      else ++waves;
    }
    const double regs = (double)src->regs();
    const double outs = regs / (double)(int64_t(1) << inLane);
    f["valu_issues"] += regs - outs;
    f["reduction_shuffles"] += outs * lanes;
    if (waves) {
      f["conversion_bytes"] += 2.0 * outs * 64 * src->waves() * 4;
      f["barriers"] += 1.0;
    }
    return true;
  }

  bool costElementwise(Operation* op, const std::vector<int64_t>& asg, Features& f) {
    if (!op->numResults() || !op->result(0).type().isTensor()) return true;
    auto l = classLayout(classOf(op->result(0)), asg);
    if (!l) return false;
    f[isTranscendental(op) ? "trans_issues" : "valu_issues"] += (double)l->regs();
    return true;
  }

  bool costBroadcast(Operation* op, const std::vector<int64_t>& asg, Features& f, std::vector<std::string>* conv) {
    auto out = classLayout(classOf(op->result(0)), asg);
    auto in = classLayout(classOf(op->operand(0)), asg);
    if (!out || !in) return false;
    const auto dims = op->attr("dimensions");
    int axis = 1;
    if (dims && dims.kind() == AttrKind::DenseI64Array && !dims->ints.empty()) axis = (int)dims->ints[0];
    if (*in != sliceLayout(*out, axis)) addConversion(op, 0, op->operand(0), f, conv);
    return true;
  }

  // Global accesses of a tile: 128-byte lines per wave instruction.
  double globalLines(Type memTy, const DistLayout& l) {
    const int64_t eb = elemBytes(memTy.elementType());
    const int64_t ld = memTy.dim(memTy.rank() - 1);
    int vb = 0;
    while (vb < l.regBits && l.basis[vb][0] == 0 && l.basis[vb][1] == (int64_t(1) << vb)) ++vb;
    const int64_t vecElems = std::min<int64_t>(int64_t(1) << vb, 16 / eb);
    double lines = 0;
    for (int64_t wv = 0; wv < l.waves(); ++wv)
      for (int64_t ins = 0; ins < l.regs() / vecElems; ++ins) {
        std::set<int64_t> seen;
        for (int64_t lane = 0; lane < 64; ++lane) {
          auto rc = l.at(ins * vecElems, lane, wv);
          const int64_t a0 = (rc[0] * ld + rc[1]) * eb;
          seen.insert(a0 / 128);
          seen.insert((a0 + vecElems * eb - 1) / 128);
        }
        lines += (double)seen.size();
      }
    return lines;
  }

  bool costTile(Operation* op, const std::vector<int64_t>& asg, Features& f) {
    const bool store = op->is("frisk.tile_store");
    Value tensor = store ? op->operand(0) : op->result(0);
    Value mem = store ? op->operand(1) : op->operand(0);
    auto l = classLayout(classOf(tensor), asg);
    if (!l) return false;
    const std::string key = "tile" + std::to_string((uintptr_t)op) + ":" + layoutKey(*l) + ":" +
                            std::to_string(storageChoice(mem, asg));
    if (auto it = memo_.find(key); it != memo_.end()) {
      f[mem.type().memorySpaceInt() == 3 ? (store ? "lds_write_cycles" : "lds_read_cycles") : "global_lines"] +=
          it->second;
      return true;
    }
    if (mem.type().memorySpaceInt() == 3) {
      const int ri = storageRootOf(rootMemref(mem));
      if (ri >= 0 && asg[roots_[ri].var] < 0) return false;
      const int64_t eb = elemBytes(mem.type().elementType());
      double c = 0;
      for (int64_t wv = 0; wv < l->waves(); ++wv)
        for (int64_t reg = 0; reg < l->regs(); ++reg) {
          std::vector<int64_t> addrs(64);
          for (int64_t lane = 0; lane < 64; ++lane) {
            auto rc = l->at(reg, lane, wv);
            addrs[lane] = ldsAddress(mem, rc[0], l->rank == 2 ? rc[1] : 0, asg);
          }
          c += ldsCycles(addrs, std::max<int64_t>(4, eb));
        }
      memo_[key] = c;
      f[store ? "lds_write_cycles" : "lds_read_cycles"] += c;
    } else {
      const double lines = globalLines(mem.type(), *l);
      memo_[key] = lines;
      f["global_lines"] += lines;
    }
    return true;
  }

  // A whole-tile copy global -> LDS runs with 16 B per lane, row-major.
  bool costCopy(Operation* op, const std::vector<int64_t>& asg, Features& f) {
    Value dst = op->operand(1);
    Type dt = dst.type();
    if (!dt.isMemRef() || dt.memorySpaceInt() != 3 || dt.rank() != 2) return true;
    const int ri = storageRootOf(rootMemref(dst));
    if (ri >= 0 && asg[roots_[ri].var] < 0) return false;
    const std::string key = "copy" + std::to_string((uintptr_t)op) + ":" + std::to_string(storageChoice(dst, asg));
    if (auto it = memo_.find(key); it != memo_.end()) {
      f["lds_write_cycles"] += it->second;
      f["global_lines"] += (double)dt.numElements() * elemBytes(dt.elementType()) / 128.0;
      return true;
    }
    const int64_t eb = elemBytes(dt.elementType());
    const int64_t threads = threadsOf_.count(op) ? threadsOf_[op] : 128;
    const int64_t vec = std::min<int64_t>(16 / eb, dt.dim(1));
    auto l = blockedLayout(dt.dim(0), dt.dim(1), 2, threads, vec);
    if (!l) return true;
    double c = 0;
    for (int64_t wv = 0; wv < l->waves(); ++wv)
      for (int64_t ins = 0; ins < l->regs() / vec; ++ins) {
        std::vector<int64_t> addrs(64);
        for (int64_t lane = 0; lane < 64; ++lane) {
          auto rc = l->at(ins * vec, lane, wv);
          addrs[lane] = ldsAddress(dst, rc[0], rc[1], asg);
        }
        c += ldsCycles(addrs, vec * eb);
      }
    memo_[key] = c;
    f["lds_write_cycles"] += c;
    f["global_lines"] += (double)dt.numElements() * eb / 128.0;
    return true;
  }

  // Cost of an assignment; `complete` is false when some term could not be
  // evaluated (partial assignment).
  double evaluate(const std::vector<int64_t>& asg, Features& f, bool& complete,
                  std::vector<std::string>* conv = nullptr) {
    layouts_.assign(classes_.size(), std::nullopt);
    complete = true;
    for (Operation* op : ops_) {
      bool ok = true;
      if (op->is("frisk.mma")) {
        for (auto& s : mmas_)
          if (s.op == op) ok = costMma(s, asg, f, conv);
      } else if (op->is("frisk.reduce_tensor")) {
        ok = costReduce(op, asg, f);
      } else if (op->is("linalg.broadcast")) {
        ok = costBroadcast(op, asg, f, conv);
      } else if (op->is("frisk.tile_store") || op->is("frisk.tile_load")) {
        ok = costTile(op, asg, f);
      } else if (op->is("frisk.copy")) {
        ok = costCopy(op, asg, f);
      } else if (isElementwise(op)) {
        ok = costElementwise(op, asg, f);
      }
      complete &= ok;
    }
    double share = 1.0;
    if (opts_.profile.simdShare) {
      int64_t threads = 0;
      for (auto& kv : threadsOf_) threads = std::max(threads, kv.second);
      share = (threads > 0 ? threads : 128) / 64.0 / 4.0;
    }
    const auto& perWave = CostProfile::perWaveFeatures();
    double total = 0;
    for (auto& kv : f) {
      auto w = opts_.profile.weights.find(kv.first);
      const double scale =
          std::find(perWave.begin(), perWave.end(), kv.first) != perWave.end() ? share : 1.0;
      total += (w == opts_.profile.weights.end() ? 0.0 : w->second) * kv.second * scale;
    }
    return total;
  }

  // ---- search -------------------------------------------------------------
  void solve() {
    const size_t nv = vars_.size();
    // Domain product (saturating).
    int64_t product = 1;
    bool overflow = false;
    for (auto& v : vars_) {
      if (v.domain <= 0) {
        rep_.failure = "empty-domain: " + v.name;
        return;
      }
      if (product > std::numeric_limits<int64_t>::max() / v.domain) overflow = true;
      else product *= v.domain;
    }
    rep_.combinations = overflow ? -1 : product;
    std::vector<int64_t> asg(nv, -1);
    double bestCost = std::numeric_limits<double>::infinity();
    if (!overflow && product <= opts_.exactCombinationLimit) {
      rep_.method = "exact";
      std::vector<int64_t> cur(nv, 0);
      for (int64_t it = 0; it < product; ++it) {
        int64_t x = it;
        for (size_t i = 0; i < nv; ++i) {
          cur[i] = x % vars_[i].domain;
          x /= vars_[i].domain;
        }
        Features f;
        bool complete;
        const double c = evaluate(cur, f, complete);
        ++rep_.expanded;
        if (c < bestCost - 1e-9) {
          bestCost = c;
          best_ = cur;
        }
      }
    } else {
      rep_.method = "beam";
      struct State {
        std::vector<int64_t> asg;
        double cost;
      };
      std::vector<State> beam = {{asg, 0.0}};
      for (size_t v = 0; v < nv; ++v) {
        std::vector<State> next;
        for (const State& s : beam)
          for (int64_t c = 0; c < vars_[v].domain; ++c) {
            if (++rep_.expanded > opts_.maxExpandedStates) {
              rep_.failure = "search-budget: more than " + std::to_string(opts_.maxExpandedStates) +
                             " expanded states";
              return;
            }
            State t = s;
            t.asg[v] = c;
            Features f;
            bool complete;
            t.cost = evaluate(t.asg, f, complete);
            next.push_back(std::move(t));
          }
        std::stable_sort(next.begin(), next.end(), [](const State& a, const State& b) { return a.cost < b.cost; });
        if ((int64_t)next.size() > opts_.beamWidth) next.resize(opts_.beamWidth);
        beam = std::move(next);
      }
      if (beam.empty()) {
        rep_.failure = "search-incomplete";
        return;
      }
      best_ = beam.front().asg;
      Features f;
      bool complete;
      bestCost = evaluate(best_, f, complete);
    }
    if (best_.empty() && nv) {
      rep_.failure = "search-incomplete";
      return;
    }
    Features f;
    bool complete = true;
    std::vector<std::string> conv;
    rep_.cost = evaluate(best_, f, complete, &conv);
    if (!complete) {
      rep_.failure = "verification: an operation's layout is undetermined";
      return;
    }
    // Classes no cost term consulted (a value nothing reads, such as an
    // unused MMA result) are resolved from the chosen assignment here.
    for (size_t c = 0; c < classes_.size(); ++c) classLayout((int)c, best_);
    rep_.features = f;
    rep_.conversions = conv;
    for (size_t i = 0; i < nv; ++i) {
      const Var& v = vars_[i];
      std::string choice;
      if (v.kind == VarKind::Mma) choice = mmas_[v.index].bindings[best_[i]].str();
      else if (v.kind == VarKind::Storage) choice = roots_[v.index].cands[best_[i]].str(roots_[v.index].rowBytes);
      else choice = classes_[v.index].freeCands[best_[i]].str();
      rep_.assignments.push_back(v.name + ": " + choice);
    }
    verifySolution();
    rep_.status = "solved";
  }

  void verifySolution() {
    for (size_t c = 0; c < classes_.size(); ++c) {
      auto l = layouts_[c];
      if (!l) throw InvalidArgument("layout-inference: verification: value#" + std::to_string(c) + " has no layout");
      if (!l->coversTile())
        throw InvalidArgument("layout-inference: verification: value#" + std::to_string(c) +
                              " layout leaves tile elements without an owner");
      if (l->rows != classes_[c].rows || l->cols != classes_[c].cols)
        throw InvalidArgument("layout-inference: verification: value#" + std::to_string(c) + " layout shape mismatch");
    }
  }

  // ---- materialization ----------------------------------------------------
  void materialize() {
    Context* ctx = mod_->ctx;
    Type i64 = ctx->integer(64);
    // Layout of every tensor-producing op result.
    for (Operation* op : ops_) {
      for (unsigned i = 0; i < op->numResults(); ++i) {
        const int c = classOf(op->result(i));
        if (c < 0) continue;
        op->setAttr(i == 0 ? "frisk.layout" : "frisk.layout_" + std::to_string(i),
                    Attribute::opaque(layouts_[c]->str()));
      }
    }
    for (auto& s : mmas_) {
      const MmaBinding& b = s.bindings[best_[s.var]];
      const bool aMem = s.op->operand(0).type().isMemRef(), bMem = s.op->operand(1).type().isMemRef();
      s.op->setAttr("form", Attribute::string(std::string(aMem ? "s" : "r") + (bMem ? "s" : "r")));
      s.op->setAttr("frisk.execution_threads", Attribute::integer(i64, s.threads));
      s.op->setAttr("frisk.mma_contract", Attribute::opaque("#frisk.mma_contract<" + b.str() + ">"));
    }
    for (Operation* op : ops_) {
      if (!op->is("frisk.reduce_tensor")) continue;
      const DistLayout& src = *layouts_[classOf(op->operand(0))];
      const int axis = (int)op->intAttr("dim");
      std::vector<int> regs, lanes, waves;
      for (int i = 0; i < src.carrierBits(); ++i) {
        if (src.basis[i][axis] == 0) continue;
        if (i < src.regBits) regs.push_back(i);
        else if (i < src.regBits + 6) lanes.push_back(i - src.regBits);
        else waves.push_back(i - src.regBits - 6);
      }
      auto list = [](const std::vector<int>& v) {
        std::ostringstream os;
        os << '[';
        for (size_t i = 0; i < v.size(); ++i) os << (i ? ", " : "") << (1 << v[i]);
        os << ']';
        return os.str();
      };
      std::ostringstream os;
      os << "#frisk.reduction_contract<{dim = " << axis << ", register_masks = " << list(regs)
         << ", lane_xor_masks = " << list(lanes) << ", wave_xor_masks = " << list(waves) << "}>";
      op->setAttr("frisk.reduction_contract", Attribute::opaque(os.str()));
      if (threadsOf_.count(op)) op->setAttr("frisk.execution_threads", Attribute::integer(i64, threadsOf_[op]));
    }
    for (auto& r : roots_) {
      if (Operation* d = r.root.definingOp())
        d->setAttr("frisk.storage", Attribute::opaque(r.cands[best_[r.var]].str(r.rowBytes)));
    }
    for (Operation* op : ops_)
      if (op->is("frisk.layout_view")) {
        const int ri = storageRootOf(rootMemref(op->operand(0)));
        if (ri >= 0) op->setAttr("frisk.storage", Attribute::opaque(roots_[ri].cands[best_[roots_[ri].var]].str(roots_[ri].rowBytes)));
      }
    // Conversions: a frisk.convert_layout in front of each mismatched use.
    for (auto& s : mmas_) {
      const MmaBinding& b = s.bindings[best_[s.var]];
      for (unsigned w = 0; w < 3; ++w) {
        Value v = s.op->operand(w);
        if (!v.type().isTensor()) continue;
        if (w == 2 && v.definingOp() && v.definingOp()->is("arith.constant")) continue;
        const char which = w == 0 ? 'A' : w == 1 ? 'B' : 'C';
        DistLayout req = mmaOperandLayout(s, b, which);
        const DistLayout& have = *layouts_[classOf(v)];
        bool ok = have == req;
        if (!ok && w < 2 && s.op->operand(1 - w).type().isMemRef()) {
          const int kAxis = (which == 'A') != (which == 'A' ? s.ta : s.tb) ? 1 : 0;
          ok = equalUpToAxisPermutation(have, req, kAxis);
        }
        if (!ok) insertConversion(s.op, w, have, req);
      }
    }
    for (Operation* op : ops_) {
      if (!op->is("linalg.broadcast")) continue;
      const auto dims = op->attr("dimensions");
      int axis = 1;
      if (dims && dims.kind() == AttrKind::DenseI64Array && !dims->ints.empty()) axis = (int)dims->ints[0];
      const DistLayout& out = *layouts_[classOf(op->result(0))];
      const DistLayout& in = *layouts_[classOf(op->operand(0))];
      if (in != sliceLayout(out, axis)) insertConversion(op, 0, in, sliceLayout(out, axis));
    }
    mod_->setAttr("frisk.layout_cost_model", Attribute::string(opts_.profile.id));
    rep_.status = "materialized";
  }

  void insertConversion(Operation* user, unsigned operand, const DistLayout& from, const DistLayout& to) {
    Value v = user->operand(operand);
    Builder b(user->ctx);
    b.setInsertionPoint(user);
    b.setLoc(user->loc);
    Operation* cv = b.create("frisk.convert_layout", {v}, {v.type()},
                             {{"source", Attribute::opaque(from.str())}, {"target", Attribute::opaque(to.str())}});
    cv->setAttr("frisk.layout", Attribute::opaque(to.str()));
    user->setOperand(operand, cv->result(0));
    ++rep_.conversionsInserted;
  }
};

}  // namespace

InferReport inferLayouts(Operation* module, const InferOptions& opts) {
  if (!module || !module->is("builtin.module")) throw InvalidArgument("layout-inference: expected a module");
  if (opts.exactCombinationLimit < 0 || opts.beamWidth <= 0 || opts.maxExpandedStates <= 0)
    throw InvalidArgument("layout-inference: solver limits must be positive");
  Inference inf(module, opts);
  return inf.run();
}

// ============================================================================
// Execution export
// ============================================================================
namespace {

std::optional<DistLayout> parseEncoding(const std::string& s) {
  // #frisk.distributed<tile = [R(, C)], topology = [regs, 64, waves],
  //   reg = [[r, c], ...], lane = [...], wave = [...]>
  auto grabList = [&](const std::string& key, size_t from) -> std::pair<std::vector<int64_t>, size_t> {
    size_t p = s.find(key + " = [", from);
    if (p == std::string::npos) return {{}, std::string::npos};
    p += key.size() + 4;
    int depth = 1;
    size_t q = p;
    while (q < s.size() && depth) {
      if (s[q] == '[') ++depth;
      if (s[q] == ']') --depth;
      ++q;
    }
    std::vector<int64_t> nums;
    std::string cur;
    for (size_t i = p; i < q - 1; ++i) {
      if (isdigit((unsigned char)s[i]) || s[i] == '-') cur += s[i];
      else if (!cur.empty()) {
        nums.push_back(std::stoll(cur));
        cur.clear();
      }
    }
    if (!cur.empty()) nums.push_back(std::stoll(cur));
    return {nums, q};
  };
  auto tile = grabList("tile", 0);
  auto topo = grabList("topology", 0);
  auto reg = grabList("reg", 0);
  auto lane = grabList("lane", 0);
  auto wave = grabList("wave", 0);
  if (tile.second == std::string::npos || topo.first.size() != 3) return std::nullopt;
  DistLayout l;
  l.rank = (int)tile.first.size();
  l.rows = tile.first[0];
  l.cols = l.rank == 2 ? tile.first[1] : 1;
  l.regBits = log2i(topo.first[0]);
  l.waveBits = log2i(topo.first[2]);
  for (auto* part : {&reg.first, &lane.first, &wave.first})
    for (size_t i = 0; i + 1 < part->size(); i += 2) l.basis.push_back({(*part)[i], (*part)[i + 1]});
  if ((int)l.basis.size() != l.carrierBits()) return std::nullopt;
  return l;
}

std::string jsonEscape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    o += c;
  }
  return o;
}

std::string ints(const std::vector<int64_t>& v) {
  std::ostringstream os;
  os << '[';
  for (size_t i = 0; i < v.size(); ++i) os << (i ? "," : "") << v[i];
  os << ']';
  return os.str();
}

}  // namespace

std::string exportExecution(Operation* module, std::string* error) {
  auto fail = [&](const std::string& m) {
    if (error) *error = m;
    return std::string();
  };
  if (!module || !module->is("builtin.module")) return fail("export: expected a module");
  Attribute t = module->attr("frisk.target");
  if (!t || t.kind() != AttrKind::String || t->s != "gfx950") return fail("export: requires frisk.target = \"gfx950\"");
  if (!module->attr("frisk.layout_cost_model")) return fail("export: layouts are not materialized (run infer_layouts)");
  std::unordered_map<ValueImpl*, int64_t> ids;
  std::vector<Value> values;
  auto id = [&](Value v) {
    auto it = ids.find(v.impl());
    if (it != ids.end()) return it->second;
    const int64_t n = (int64_t)ids.size();
    ids[v.impl()] = n;
    values.push_back(v);
    return n;
  };
  std::unordered_map<ValueImpl*, std::string> encodings;  // tensor value -> distributed encoding
  std::unordered_map<ValueImpl*, std::string> storages;   // memref value -> storage encoding
  std::ostringstream ops;
  bool firstOp = true;
  std::string err;
  std::function<void(Operation*)> emit = [&](Operation* op) {
    for (auto& r : op->regions)
      for (auto& blk : r->blocks)
        for (unsigned i = 0; i < blk->numArguments(); ++i) id(blk->argument(i));
    std::vector<int64_t> in, out;
    for (Value v : op->operands) in.push_back(id(v));
    for (unsigned i = 0; i < op->numResults(); ++i) {
      out.push_back(id(op->result(i)));
      Attribute a = op->attr(i == 0 ? "frisk.layout" : "frisk.layout_" + std::to_string(i));
      if (a && op->result(i).type().isTensor()) encodings[op->result(i).impl()] = a->s;
      if (Attribute s = op->attr("frisk.storage"); s && op->result(i).type().isMemRef())
        storages[op->result(i).impl()] = s->s;
      if (op->result(i).type().isTensor() && !a && err.empty() && op->parentOp() &&
          !op->is("arith.constant") && !op->is("tensor.empty"))
        err = "export: " + op->name + " result has no materialized layout";
    }
    ops << (firstOp ? "" : ",") << "\n  {\"name\": \"" << op->name << "\", \"operands\": " << ints(in)
        << ", \"results\": " << ints(out);
    if (op->numRegions()) {
      ops << ", \"region_args\": [";
      bool fb = true;
      for (auto& r : op->regions)
        for (auto& blk : r->blocks) {
          std::vector<int64_t> args;
          for (unsigned i = 0; i < blk->numArguments(); ++i) args.push_back(id(blk->argument(i)));
          ops << (fb ? "" : ",") << ints(args);
          fb = false;
        }
      ops << "]";
    }
    ops << ", \"attrs\": {";
    firstOp = false;
    bool fa = true;
    for (auto& na : op->attrs) {
      ops << (fa ? "" : ", ") << '"' << jsonEscape(na.name) << "\": ";
      const Attribute& a = na.value;
      if (a.kind() == AttrKind::Integer) ops << a->i;
      else if (a.kind() == AttrKind::Bool) ops << (a->b ? "true" : "false");
      else if (a.kind() == AttrKind::String || a.kind() == AttrKind::Opaque) ops << '"' << jsonEscape(a->s) << '"';
      else if (a.kind() == AttrKind::DenseI64Array) ops << ints(a->ints);
      else ops << '"' << jsonEscape(a.str()) << '"';
      fa = false;
    }
    ops << "}";
    if (op->is("frisk.reduce_tensor")) {
      // Reduction fibers: for each output element, the (reg, lane, wave)
      // holders of the source elements it combines, in carrier order.
      auto it = encodings.find(op->operand(0).impl());
      std::optional<DistLayout> src;
      if (it != encodings.end()) src = parseEncoding(it->second);
      if (!src) {
        if (err.empty()) err = "export: reduce_tensor source has no layout";
      } else {
        const int axis = (int)op->intAttr("dim");
        const int64_t outN = axis == 1 ? src->rows : src->cols;
        std::vector<std::vector<int64_t>> fibers(outN);
        const uint64_t carriers = uint64_t(1) << src->carrierBits();
        std::vector<std::set<int64_t>> seen(outN);
        for (uint64_t c = 0; c < carriers; ++c) {
          auto rc = src->at(c);
          const int64_t o = axis == 1 ? rc[0] : rc[1];
          const int64_t e = axis == 1 ? rc[1] : rc[0];
          if (seen[o].insert(e).second) fibers[o].push_back((int64_t)c);
        }
        ops << ", \"fibers\": [";
        for (int64_t o = 0; o < outN; ++o) ops << (o ? "," : "") << ints(fibers[o]);
        ops << "], \"carrier\": [\"reg\", \"lane\", \"wave\"], \"topology\": "
            << ints({src->regs(), 64, src->waves()});
      }
    }
    ops << "}";
    for (auto& r : op->regions)
      for (auto& blk : r->blocks)
        for (auto& o : blk->ops) emit(o.get());
  };
  for (auto& r : module->regions)
    for (auto& blk : r->blocks)
      for (auto& o : blk->ops) emit(o.get());
  if (!err.empty()) return fail(err);
  std::ostringstream vs;
  bool firstV = true;
  for (Value v : values) {
    vs << (firstV ? "" : ",") << "\n  {\"id\": " << ids[v.impl()] << ", \"type\": \"" << jsonEscape(v.type().str()) << '"';
    firstV = false;
    auto e = encodings.find(v.impl());
    if (e != encodings.end()) {
      auto l = parseEncoding(e->second);
      if (!l) return fail("export: unreadable layout " + e->second);
      const uint64_t carriers = uint64_t(1) << l->carrierBits();
      std::vector<int64_t> logical(carriers), first(l->rows * l->cols, -1);
      for (uint64_t c = 0; c < carriers; ++c) {
        auto rc = l->at(c);
        const int64_t idx = rc[0] * l->cols + rc[1];
        logical[c] = idx;
        if (first[idx] < 0) first[idx] = (int64_t)c;
      }
      vs << ", \"distributed\": {\"encoding\": \"" << jsonEscape(e->second) << "\", \"topology\": "
         << ints({l->regs(), 64, l->waves()}) << ", \"shape\": "
         << ints(l->rank == 2 ? std::vector<int64_t>{l->rows, l->cols} : std::vector<int64_t>{l->rows})
         << ", \"replication\": " << l->replication() << ", \"logical\": " << ints(logical)
         << ", \"first\": " << ints(first) << "}";
    }
    auto s = storages.find(v.impl());
    if (s != storages.end()) {
      Type mt = v.type();
      vs << ", \"storage\": {\"layout\": \"" << jsonEscape(s->second) << "\"";
      // Byte offset of every element of a rank-2 LDS tile under the swizzle.
      if (mt.rank() == 2 && mt.hasStaticShape()) {
        const int64_t eb = std::max<int64_t>(1, mt.elementType().bitWidth() / 8);
        const int64_t rowBytes = mt.dim(1) * eb;
        std::optional<SwizzleProposal> swz;
        const std::string& txt = s->second;
        const size_t p = txt.find("swizzle = \"");
        std::string formula = p == std::string::npos ? "c" : txt.substr(p + 11, txt.find('"', p + 11) - p - 11);
        if (formula != "c" && isPow2(rowBytes) && rowBytes >= 32) {
          for (int atom : {32, 16}) {
            SwizzleProposal q = proposeLdsSwizzle(rowBytes, atom);
            if (q.formula == formula) swz = q;
          }
          if (!swz) return fail("export: unknown swizzle " + formula);
        }
        std::vector<int64_t> offs;
        for (int64_t r = 0; r < mt.dim(0); ++r)
          for (int64_t c = 0; c < mt.dim(1); ++c) offs.push_back(swz ? swz->offset(r, c * eb) : r * rowBytes + c * eb);
        vs << ", \"row_bytes\": " << rowBytes << ", \"byte_offsets\": " << ints(offs);
      }
      vs << "}";
    }
    vs << "}";
  }
  std::ostringstream out;
  out << "{\"schema_version\": 1, \"target\": \"gfx950\", \"cost_model\": \""
      << jsonEscape(module->attr("frisk.layout_cost_model")->s) << "\",\n \"values\": [" << vs.str()
      << "\n ],\n \"operations\": [" << ops.str() << "\n ]}\n";
  return out.str();
}

}  // namespace fir
