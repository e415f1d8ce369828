// CDNA4 layout target: MFMA table, tile-product geometry, fragment maps
// (checked GF(2) linear forms) and LDS swizzle proposals.
#include "layout.h"

#include "../csrc/launch_plan.h"

#include <algorithm>
#include <cmath>
#include <sstream>
#include <unordered_map>

namespace fir {

namespace {
bool isPow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int log2i(int64_t x) {
  int b = 0;
  while ((int64_t(1) << b) < x) ++b;
  return b;
}
}  // namespace

// Dense MFMA shapes of gfx950 used by the kernels (wave64; every lane holds
// m*k/64 inputs of A and of B and m*n/64 accumulators).
const std::vector<MfmaInstr>& cdna4MfmaTable() {
  static const std::vector<MfmaInstr> table = {
      {"v_mfma_f32_32x32x16_f16", MfmaInput::F16, 32, 32, 16, 32, 16},
      {"v_mfma_f32_16x16x32_f16", MfmaInput::F16, 16, 16, 32, 32, 16},
      {"v_mfma_f32_32x32x16_bf16", MfmaInput::BF16, 32, 32, 16, 32, 16},
      {"v_mfma_f32_16x16x32_bf16", MfmaInput::BF16, 16, 16, 32, 32, 16},
      {"v_mfma_f32_32x32x64_f8f6f4", MfmaInput::FP8, 32, 32, 64, 32, 8},
      {"v_mfma_f32_16x16x128_f8f6f4", MfmaInput::FP8, 16, 16, 128, 32, 8},
      {"v_mfma_i32_32x32x32_i8", MfmaInput::I8, 32, 32, 32, 32, 8},
      {"v_mfma_i32_16x16x64_i8", MfmaInput::I8, 16, 16, 64, 32, 8},
      {"v_mfma_f32_32x32x2_f32", MfmaInput::F32, 32, 32, 2, 32, 32},
      {"v_mfma_f32_16x16x4_f32", MfmaInput::F32, 16, 16, 4, 32, 32},
  };
  return table;
}

std::optional<MfmaInput> mfmaInputOf(Type e) {
  if (e.isF16()) return MfmaInput::F16;
  if (e.isBF16()) return MfmaInput::BF16;
  if (e.isFloat(FloatKind::E4M3FN) || e.isFloat(FloatKind::E5M2)) return MfmaInput::FP8;
  if (e.isSignlessInteger(8)) return MfmaInput::I8;
  if (e.isF32()) return MfmaInput::F32;
  return std::nullopt;
}

std::optional<MmaGeometry> cdna4MmaGeometry(int64_t m, int64_t n, int64_t k, Type in, Type acc,
                                            int64_t threads, GemmWarpPolicy policy) {
  auto kind = mfmaInputOf(in);
  if (!kind || policy == GemmWarpPolicy::Auto) return std::nullopt;
  const bool accOk = *kind == MfmaInput::I8 ? acc.isSignlessInteger(32) : acc.isF32();
  if (!accOk || threads < 64 || threads > 1024 || !isPow2(threads)) return std::nullopt;
  if (m <= 0 || n <= 0 || k <= 0) return std::nullopt;
  const int64_t waves = threads / 64;
  std::optional<MmaGeometry> best;
  int64_t bestScore = 0;
  for (int64_t gM = 1; gM <= waves; gM *= 2) {
    const int64_t gN = waves / gM;
    if (m % gM || n % gN) continue;
    const int64_t wm = m / gM, wn = n / gN;
    const MfmaInstr* atom = nullptr;
    for (const MfmaInstr& ins : cdna4MfmaTable()) {  // 32x32 before 16x16
      if (ins.input != *kind) continue;
      if (wm % ins.m == 0 && wn % ins.n == 0 && k % ins.k == 0) {
        atom = &ins;
        break;
      }
    }
    if (!atom) continue;
    int64_t score = std::llabs(wm - wn);
    if (policy == GemmWarpPolicy::FullRow) score = -gM;
    if (policy == GemmWarpPolicy::FullCol) score = -gN;
    if (!best || score < bestScore) {
      best = MmaGeometry{m, n, k, threads, gM, gN, *atom, wm / atom->m, wn / atom->n, k / atom->k};
      bestScore = score;
    }
  }
  return best;
}

// Atom-level maps.  A: lane L holds row L % am at k = (ak/groups) * (L / am)
// + e with groups = 64 / am; B mirrors A with columns; C (32x32): element e
// of lane L is row 8 (e/4) + 4 (L/32) + e%4, column L%32; C (16x16): row
// 4 (L/16) + e, column L%16.  The A/B k assignment is the one the GEMM and
// attention kernels feed the instruction with (A and B share it, so a
// product does not depend on the instruction's internal k order).
std::array<int64_t, 2> cdna4FragmentCoordinate(const MmaGeometry& g, char operand, int64_t reg,
                                               int64_t lane, int64_t wave) {
  const MfmaInstr& a = g.atom;
  const int64_t wm = wave / g.gN, wn = wave % g.gN;
  const int64_t groups = 64 / a.m;
  if (operand == 'C') {
    const int64_t per = g.cPerLane();
    const int64_t e = reg % per, blk = reg / per;
    const int64_t i = blk / g.nRepeat, j = blk % g.nRepeat;
    int64_t r, c;
    if (a.m == 32) {
      r = 8 * (e / 4) + 4 * (lane / 32) + e % 4;
      c = lane % 32;
    } else {
      r = 4 * (lane / 16) + e;
      c = lane % 16;
    }
    return {wm * (g.m / g.gM) + i * a.m + r, wn * (g.n / g.gN) + j * a.n + c};
  }
  const int64_t per = g.aPerLane();
  const int64_t e = reg % per, blk = reg / per;
  const int64_t outer = blk / g.kRepeat, kk = blk % g.kRepeat;
  const int64_t kIn = (a.k / groups) * (lane / a.m) + e;
  const int64_t mn = lane % a.m;
  if (operand == 'A') return {wm * (g.m / g.gM) + outer * a.m + mn, kk * a.k + kIn};
  return {kk * a.k + kIn, wn * (g.n / g.gN) + outer * a.n + mn};
}

uint64_t Gf2Map::apply(uint64_t x) const {
  uint64_t y = 0;
  for (int i = 0; i < inBits; ++i)
    if ((x >> i) & 1) y ^= cols[i];
  return y;
}

int Gf2Map::rank() const {
  std::vector<uint64_t> v = cols;
  int r = 0;
  for (int bit = 0; bit < outBits; ++bit) {
    auto it = std::find_if(v.begin() + r, v.end(), [&](uint64_t c) { return (c >> bit) & 1; });
    if (it == v.end()) continue;
    std::swap(*it, v[r]);
    for (size_t j = 0; j < v.size(); ++j)
      if ((int)j != r && ((v[j] >> bit) & 1)) v[j] ^= v[r];
    ++r;
  }
  return r;
}

std::optional<Gf2Map> cdna4FragmentGf2(const MmaGeometry& g, char operand) {
  const int64_t regs = operand == 'A' ? g.aRegs() : operand == 'B' ? g.bRegs() : g.cRegs();
  const int64_t rows = operand == 'B' ? g.k : g.m;
  const int64_t cols = operand == 'A' ? g.k : g.n;
  if (!isPow2(regs) || !isPow2(rows) || !isPow2(cols) || !isPow2(g.waves())) return std::nullopt;
  const int rb = log2i(regs), wb = log2i(g.waves()), rowBits = log2i(rows);
  Gf2Map map;
  map.inBits = rb + 6 + wb;
  map.outBits = rowBits + log2i(cols);
  auto eval = [&](uint64_t x) {
    const int64_t reg = x & (regs - 1), lane = (x >> rb) & 63, wave = x >> (rb + 6);
    auto rc = cdna4FragmentCoordinate(g, operand, reg, lane, wave);
    return (uint64_t)rc[0] | ((uint64_t)rc[1] << rowBits);
  };
  for (int i = 0; i < map.inBits; ++i) map.cols.push_back(eval(uint64_t(1) << i));
  if (eval(0) != 0) return std::nullopt;
  for (uint64_t x = 0; x < (uint64_t(1) << map.inBits); ++x)
    if (eval(x) != map.apply(x)) return std::nullopt;
  return map;
}

double ldsReadB128ConflictFactor(const std::vector<int64_t>& addrs) {
  int64_t total = 0, phases = 0;
  for (size_t p = 0; p < addrs.size(); p += 16, ++phases) {
    std::unordered_map<int64_t, std::vector<int64_t>> banks;
    for (size_t l = p; l < std::min(addrs.size(), p + 16); ++l)
      for (int w = 0; w < 4; ++w) {
        const int64_t dw = addrs[l] / 4 + w;
        auto& v = banks[dw % 64];
        if (std::find(v.begin(), v.end(), dw) == v.end()) v.push_back(dw);
      }
    size_t worst = 0;
    for (auto& kv : banks) worst = std::max(worst, kv.second.size());
    total += (int64_t)worst;
  }
  return phases ? (double)total / (double)phases : 1.0;
}

int64_t SwizzleProposal::chunk(int64_t row, int64_t c) const {
  int64_t f = 0;
  for (auto& t : terms) f ^= ((row >> t.shift) & t.mask) << t.lshift;
  return (c ^ f) & (rowBytes / 16 - 1);
}

int64_t SwizzleProposal::offset(int64_t row, int64_t byte) const {
  return row * rowBytes + chunk(row, byte / 16) * 16 + byte % 16;
}

SwizzleProposal proposeLdsSwizzle(int64_t rowBytes, int atomM) {
  if (rowBytes < 32 || !isPow2(rowBytes)) throw InvalidArgument("LDS row must be a power of two >= 32 B");
  if (atomM != 16 && atomM != 32) throw InvalidArgument("MFMA atom must be 16 or 32 rows");
  const int64_t chunks = rowBytes / 16;
  const int groups = 64 / atomM;  // lanes per row group read distinct chunks
  auto cost = [&](const SwizzleProposal& p) {
    double sum = 0;
    int n = 0;
    for (int64_t r0 = 0; r0 < 64; r0 += atomM)
      for (int64_t c0 = 0; c0 + groups <= chunks; c0 += groups) {
        std::vector<int64_t> addrs(64);
        for (int l = 0; l < 64; ++l) {
          const int64_t r = r0 + l % atomM, c = c0 + l / atomM;
          addrs[l] = r * rowBytes + p.chunk(r, c) * 16;
        }
        sum += ldsReadB128ConflictFactor(addrs);
        ++n;
      }
    return sum / n;
  };
  std::vector<SwizzleTerm> singles;
  for (int shift = 0; shift < 6; ++shift)
    for (int64_t mask = 1; mask < chunks; mask = mask * 2 + 1) singles.push_back({shift, (int)mask, 0});
  SwizzleProposal best{rowBytes, {}, 0.0, ""};
  best.readConflict = cost(best);
  auto consider = [&](std::vector<SwizzleTerm> t) {
    SwizzleProposal p{rowBytes, std::move(t), 0.0, ""};
    p.readConflict = cost(p);
    if (p.readConflict < best.readConflict - 1e-9 ||
        (std::fabs(p.readConflict - best.readConflict) < 1e-9 && p.terms.size() < best.terms.size()))
      best = p;
  };
  for (auto& s : singles) consider({s});
  if (best.readConflict > 1.0 + 1e-9)
    for (size_t i = 0; i < singles.size(); ++i)
      for (size_t j = i + 1; j < singles.size(); ++j) consider({singles[i], singles[j]});
  std::ostringstream f;
  f << "c";
  for (auto& t : best.terms) {
    f << " ^ ((r >> " << t.shift << ") & " << t.mask << ")";
    if (t.lshift) f << " << " << t.lshift;
  }
  best.formula = f.str();
  return best;
}

int64_t sm90StyleSwizzle(int64_t off, int64_t sw) {
  if (sw != 32 && sw != 64 && sw != 128) throw InvalidArgument("swizzle must be 32, 64 or 128 bytes");
  return off ^ (((off >> 7) & (sw / 16 - 1)) << 4);
}

}  // namespace fir

namespace fir {

namespace {

// frisk_dtype code of an IR element type (include/frisk_hip.h).
int dtypeCode(Type t) {
  namespace P = frisk::plan;
  if (t.isF32()) return P::kF32;
  if (t.isF16()) return P::kF16;
  if (t.isBF16()) return P::kBF16;
  if (t.isFloat(FloatKind::E4M3FN)) return P::kE4M3;
  if (t.isSignlessInteger(8)) return P::kI8;
  if (t.isSignlessInteger(32)) return P::kI32;
  throw InvalidArgument("launch contract: no GEMM kernel takes element type " + t.str());
}

}  // namespace

std::string GemmLaunchContract::str() const {
  std::ostringstream o;
  o << "#frisk.gemm_launch<{kernel = \"" << kernel << "\", tile = [" << tileM << ", " << tileN
    << "], wave_grid = [" << waveM << ", " << waveN << "], stage_bytes = " << stageBytes
    << ", slices = " << slices << ", slice_sum = \"" << sliceSum << "\"}>";
  return o.str();
}

GemmLaunchContract cdna4GemmLaunch(int64_t m, int64_t n, int64_t k, Type in, Type out, bool transA,
                                   bool transB, int64_t cus, bool workspace, bool matrixCores) {
  namespace P = frisk::plan;
  if (m <= 0 || n <= 0 || k <= 0) throw InvalidArgument("launch contract: M, N and K must be positive");
  P::GemmShape g;
  g.in = dtypeCode(in);
  g.out = dtypeCode(out);
  g.m = m;
  g.n = n;
  g.k = k;
  g.trans_a = transA;
  g.trans_b = transB;
  const P::Route r = P::route_of(g, matrixCores);
  const P::GemmLaunch L = P::launch_of(g, r, (int)cus, workspace ? INT64_MAX : 0);
  GemmLaunchContract c;
  c.kernel = L.kernel == P::Kernel::W4 ? "gemm_w4"
             : L.kernel == P::Kernel::T128 ? "gemm_128"
             : L.kernel == P::Kernel::Skinny ? "gemm_skinny" : "gemm_generic";
  c.tileM = L.tile_m;
  c.tileN = L.tile_n;
  c.waveM = L.wave_m;
  c.waveN = L.wave_n;
  c.stageBytes = L.stage_bytes;
  c.slices = L.slices;
  c.kbSlice = L.kb_slice;
  c.workspaceBytes = L.workspace_bytes;
  c.sliceSum = L.slice_sum == P::SliceSum::InLaunch ? "in_launch"
               : L.slice_sum == P::SliceSum::SecondLaunch ? "second_launch" : "none";
  if (L.kernel == P::Kernel::W4 || L.kernel == P::Kernel::T128) {
    const int es = P::dtype_bytes(g.in);
    c.swizzleA = P::lds_swizzle(transA, es, L.stage_bytes, L.tile_m * es);
    c.swizzleB = P::lds_swizzle(!transB, es, L.stage_bytes, L.tile_n * es);
  }
  return c;
}

int64_t cdna4AttentionWaves(int64_t batchHeads, int64_t seqQ, int64_t headDim, bool causal,
                            int64_t cus) {
  if (batchHeads <= 0 || seqQ <= 0) throw InvalidArgument("launch contract: sizes must be positive");
  if (headDim != 16 && headDim != 32 && headDim != 64 && headDim != 128)
    throw InvalidArgument("launch contract: the attention kernel takes head_dim 16, 32, 64 or 128");
  return frisk::plan::attn_waves(batchHeads, seqQ, headDim, causal, (int)cus);
}

}  // namespace fir
