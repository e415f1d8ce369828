// CDNA4 (gfx950) layout target: MFMA instruction table, wave-grid geometry
// of a tile matrix multiply, the (register, lane, wave) -> (row, col)
// fragment maps as GF(2) matrices, and LDS XOR-swizzle proposals.
//
// This replaces the reference's SM90 target (SM90InstructionTable.cpp:21-35,
// SM90MmaLayoutProof.cpp:25-50 and :139-153, SM90GemmConstraints.cpp:106-167)
// for 64-wide wavefronts and the MFMA shapes the GEMM / attention kernels of
// this package use.
#pragma once

#include <array>
#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "ir.h"

namespace fir {

enum class MfmaInput { F16, BF16, FP8, I8, F32 };

struct MfmaInstr {
  const char* name;   // ISA mnemonic
  MfmaInput input;
  int m, n, k;        // atom shape
  int accBits;        // 32 (f32 / i32 accumulators)
  int inBits;         // input element width
};

// All dense MFMA shapes of the table (two per input kind).
const std::vector<MfmaInstr>& cdna4MfmaTable();
std::optional<MfmaInput> mfmaInputOf(Type elem);

// Geometry of one tile product C[m, n] += A[m, k] . B[k, n] executed by
// `threads` lanes: waves = threads / 64 arranged gM x gN over (m, n); each
// wave owns an (m/gM) x (n/gN) block made of mRepeat x nRepeat atoms and
// runs kRepeat k-steps per atom.
struct MmaGeometry {
  int64_t m, n, k, threads;
  int64_t gM, gN;
  MfmaInstr atom;
  int64_t mRepeat, nRepeat, kRepeat;
  int64_t waves() const { return gM * gN; }
  // Elements per lane of one atom: A/B = atom.m * atom.k / 64; C = m*n/64.
  int64_t aPerLane() const { return (int64_t)atom.m * atom.k / 64; }
  int64_t cPerLane() const { return (int64_t)atom.m * atom.n / 64; }
  // Register (element) counts per lane over the whole wave block.
  int64_t aRegs() const { return mRepeat * kRepeat * aPerLane(); }
  int64_t bRegs() const { return nRepeat * kRepeat * aPerLane(); }
  int64_t cRegs() const { return mRepeat * nRepeat * cPerLane(); }
};

// Wave-grid choice per warp policy (Square balances the per-wave block,
// FullRow puts every wave along M, FullCol along N) and the largest atom
// that tiles the per-wave block; nullopt when no legal geometry exists.
std::optional<MmaGeometry> cdna4MmaGeometry(int64_t m, int64_t n, int64_t k, Type in, Type acc,
                                            int64_t threads, GemmWarpPolicy policy);

// (row, col) held by (reg, lane, wave) for operand 'A' (m x k), 'B' (k x n)
// or 'C' (m x n).  A is replicated over the gN waves of a wave row, B over
// the gM waves of a wave column.
std::array<int64_t, 2> cdna4FragmentCoordinate(const MmaGeometry& g, char operand, int64_t reg,
                                               int64_t lane, int64_t wave);

// A linear map over GF(2): input bits (register bits, then 6 lane bits, then
// wave bits) -> output bits (row bits, then column bits).  cols[i] is the
// image of input basis vector i.
struct Gf2Map {
  int inBits = 0, outBits = 0;
  std::vector<uint64_t> cols;
  uint64_t apply(uint64_t x) const;
  int rank() const;
};
// GF(2) form of the fragment map; nullopt if an extent is not a power of
// two or the map is not linear.
std::optional<Gf2Map> cdna4FragmentGf2(const MmaGeometry& g, char operand);

// ---- LDS -------------------------------------------------------------------
// Bank-conflict factor (1 = conflict-free) of one ds_read_b128 issued by a
// wave whose lane L reads byte address addrs[L] (16-B aligned).  Model:
// 64 banks of 4 B, lanes served 16 at a time (lanes 16p .. 16p+15 in phase
// p); a phase costs the largest number of distinct dwords mapped to one bank.
double ldsReadB128ConflictFactor(const std::vector<int64_t>& addrs);

// A row-XOR swizzle of 16-B chunks: physical chunk = c ^ f(r), with
// f(r) = XOR over terms of ((r >> shift) & mask) << lshift.
struct SwizzleTerm {
  int shift, mask, lshift;
};
struct SwizzleProposal {
  int64_t rowBytes;
  std::vector<SwizzleTerm> terms;
  double readConflict;  // modelled factor of the MFMA fragment read
  std::string formula;
  int64_t chunk(int64_t row, int64_t logicalChunk) const;
  int64_t offset(int64_t row, int64_t byteInRow) const;  // byte offset in the tile
};

// Best swizzle for reading MFMA fragments out of a row-major LDS tile with
// `rowBytes` per row: lanes 0-31 read 16 B of consecutive rows r0..r0+31 at
// one logical chunk, lanes 32-63 the next chunk (atom 32) or four 16-lane
// groups at four chunks (atom 16).  Candidates are single-term and
// two-term XORs of row bits; the cheapest modelled read wins, ties go to
// fewer terms.
SwizzleProposal proposeLdsSwizzle(int64_t rowBytes, int atomM);
// The reference's shared-memory swizzle form (attention_tile_mma.py:113-114):
// off ^ (((off >> 7) & (sw/16 - 1)) << 4) for sw in {32, 64, 128}.
int64_t sm90StyleSwizzle(int64_t off, int64_t swizzleBytes);

// ---- launch contracts ------------------------------------------------------
// The gfx950 target's launch-level decisions, shared with the C-ABI
// (frisk_amd/csrc/launch_plan.h): for a whole-matrix GEMM the kernel, its
// workgroup tile, wave grid, LDS stage depth and K split; for attention the
// waves per workgroup.  The reference binds the corresponding choice (the
// warpgroup grid of each MMA) in its SM90 layout target
// (SM90LayoutTarget.cpp:171-481).
struct GemmLaunchContract {
  std::string kernel;  // gemm_w4 (256x256), gemm_128, gemm_skinny, gemm_generic
  int64_t tileM = 0, tileN = 0, waveM = 0, waveN = 0, stageBytes = 0, slices = 1;
  int64_t kbSlice = 0, workspaceBytes = 0;
  std::string sliceSum;  // none, in_launch, second_launch
  std::string swizzleA, swizzleB;  // LDS stage-tile swizzles of the MFMA kernels
  std::string str() const;  // #frisk.gemm_launch<{...}>
};
// `workspace`: a split-K workspace is at hand; `matrixCores`: the operands
// meet the MFMA kernels' alignment and reach conditions.
GemmLaunchContract cdna4GemmLaunch(int64_t m, int64_t n, int64_t k, Type in, Type out, bool transA,
                                   bool transB, int64_t cus, bool workspace, bool matrixCores);
int64_t cdna4AttentionWaves(int64_t batchHeads, int64_t seqQ, int64_t headDim, bool causal,
                            int64_t cus);

}  // namespace fir
