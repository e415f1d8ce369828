// Layout inference for CDNA4 (gfx950): distributed layouts of tensor SSA
// values, LDS storage swizzles of shared tiles, MFMA instruction bindings of
// frisk.mma, reduction contracts, conversion edges, an additive cost model
// and the execution-packet export.
//
// Reference counterparts: the frisk-infer-layouts pass
// (lib/Dialect/Frisk/Transforms/LayoutInfer.cpp:187-282: collect constraints,
// solve exactly up to 256 combinations or by beam search of width 32 within
// 65536 expansions, verify, materialize; options include/Dialect/Frisk/
// Transforms/Passes.td:33-42), its cost model (lib/Dialect/Frisk/Target/SM90/
// SM90CostModel.cpp:302, SM90CalibratedCostModel.cpp:26-35: an additive
// integer score over named features) and frisk-export-execution
// (lib/Conversion/FriskLayoutToGPU/ExportExecution.cpp:46-295: a JSON packet
// of operations, values, distributed enumerations, storage addresses and
// reduction fibers).  Layouts here are GF(2)-linear maps from the CDNA4
// carrier (register bits, 6 lane bits, wave bits) to logical tile bits.
#pragma once

#include <array>
#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <vector>

#include "ir.h"
#include "layout.h"

namespace fir {

// A distributed layout of a rank-1 (rows x 1) or rank-2 (rows x cols) tile
// over one workgroup: carrier bit i (register bits first, then the 6 lane
// bits, then the wave bits) adds basis[i] = (row, col) under XOR.  A zero
// basis vector replicates the tile over that carrier bit.
struct DistLayout {
  int64_t rows = 1, cols = 1;
  int rank = 2;
  int regBits = 0, waveBits = 0;
  std::vector<std::array<int64_t, 2>> basis;

  int carrierBits() const { return regBits + 6 + waveBits; }
  int64_t regs() const { return int64_t(1) << regBits; }
  int64_t waves() const { return int64_t(1) << waveBits; }
  std::array<int64_t, 2> at(uint64_t carrier) const;
  std::array<int64_t, 2> at(int64_t reg, int64_t lane, int64_t wave) const {
    return at((uint64_t)reg | ((uint64_t)lane << regBits) | ((uint64_t)wave << (regBits + 6)));
  }
  int gf2Rank() const;
  bool coversTile() const;      // every logical element has an owner
  int64_t replication() const;  // owners per logical element
  std::string str() const;      // canonical textual encoding
  bool operator==(const DistLayout& o) const {
    return rows == o.rows && cols == o.cols && rank == o.rank && regBits == o.regBits &&
           waveBits == o.waveBits && basis == o.basis;
  }
  bool operator!=(const DistLayout& o) const { return !(*this == o); }
};

DistLayout transposeLayout(const DistLayout& l);
// Row-major blocked layout: vecElems consecutive columns per lane, lanes then
// waves along the row-major order, the remainder in further registers.
std::optional<DistLayout> blockedLayout(int64_t rows, int64_t cols, int rank, int64_t threads,
                                        int64_t vecElems);
// The rank-1 layout left after reducing `axis` (0 or 1) of a rank-2 layout.
DistLayout sliceLayout(const DistLayout& l, int axis);
// True when `actual` equals `required` after a linear bijection of the
// logical column index (axis 1) or row index (axis 0); the permutation's
// images of the unit vectors are returned in *perm.
bool equalUpToAxisPermutation(const DistLayout& actual, const DistLayout& required, int axis,
                              std::vector<int64_t>* perm = nullptr);

// ---- MFMA instruction bindings ------------------------------------------------
// One way to execute frisk.mma D[m, n] = A'[m, k] B'[k, n] (+ C): the MFMA
// atom, the wave grid (policy) and the orientation.  `swapped` executes the
// transposed product D^T = B'^T A'^T, so the hardware C fragment holds D
// transposed (the layout that lets a softmax result feed the next product's
// k side without a conversion).
struct MmaBinding {
  MmaGeometry hw;  // geometry of the product the MFMAs execute
  GemmWarpPolicy policy = GemmWarpPolicy::Square;
  bool swapped = false;
  // Layout of logical operand 'A' (m x k), 'B' (k x n) or 'C' (m x n).
  DistLayout operand(char which) const;
  int64_t mfmaPerWave() const { return hw.mRepeat * hw.nRepeat * hw.kRepeat; }
  std::string str() const;
};
// The MFMA bindings of an (m, n, k) product on `threads` lanes.  With the
// Auto policy every wave grid is a candidate (the solver chooses); Square,
// FullRow and FullCol fix the logical wave grid to the one that policy
// gives (SM90MmaLayoutProof.cpp:25-62: a non-Auto policy yields one
// geometry), leaving the MFMA atom and the operand orientation to the
// solver.
std::vector<MmaBinding> cdna4MmaBindings(int64_t m, int64_t n, int64_t k, Type in, Type acc,
                                         int64_t threads,
                                         GemmWarpPolicy policy = GemmWarpPolicy::Auto);

// ---- cost model ---------------------------------------------------------------
// Named features in issue cycles per wave (or bytes / barriers), weighted
// and summed: cost = sum_f weight[f] * feature[f].
struct CostProfile {
  std::string id = "cdna4-layout-v1";
  std::map<std::string, double> weights;
  // Per-wave features (MFMA, VALU, transcendental and cross-lane issue) are
  // scaled by waves / 4 before weighting: the share of a CU's four SIMDs the
  // workgroup's waves occupy, so the cost is in CU cycles per workgroup (the
  // unit a profile fitted to kernel throughput is in).
  bool simdShare = false;
  static CostProfile defaults();
  // {"id": "...", "weights": {"feature": number, ...}, "simd_share": bool,
  // "provenance": {...}}; unknown features or keys are rejected
  // (InvalidArgument), "provenance" is read past.
  static CostProfile fromJson(const std::string& text);
  static const std::vector<std::string>& featureNames();
  static const std::vector<std::string>& perWaveFeatures();
};

struct InferOptions {
  int64_t exactCombinationLimit = 256;
  int64_t beamWidth = 32;
  int64_t maxExpandedStates = 65536;
  bool analysisOnly = false;
  CostProfile profile = CostProfile::defaults();
};

struct InferReport {
  std::string status = "failed";  // "solved" (analysis only), "materialized" or "failed"
  std::string failure;
  std::string method;              // "exact" or "beam"
  std::string costModelId;
  int64_t variables = 0, combinations = 0, expanded = 0, conversionsInserted = 0;
  double cost = 0;
  std::map<std::string, double> features;
  std::vector<std::string> assignments;  // "<variable>: <choice>"
  std::vector<std::string> conversions;  // "<consumer op>#<operand>: <bytes> B"
  std::vector<std::string> graph;        // constraint listing (analysis dump)
};

// Solve and (unless analysisOnly) materialize on a module normalized by
// normalizeLegacyFragments; requires frisk.target = "gfx950".
InferReport inferLayouts(Operation* module, const InferOptions& opts);

// Execution packet (JSON) of a module whose layouts were materialized by
// inferLayouts.  Returns "" and sets *error when something is missing.
std::string exportExecution(Operation* module, std::string* error);

// Encoding strings as materialized (also used by the exporter).
std::string distributedEncoding(const DistLayout& l);

}  // namespace fir
