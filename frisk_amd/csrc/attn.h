// Flash-attention forward for gfx950 (MI355X): head_dim 16, 32, 64 or 128,
// bf16 / f16 inputs, output in the input dtype or f32.  This header holds
// the kernel template; attn_d*.hip instantiate it per head_dim (so the
// variants compile in parallel).
//
// Semantics: the attention tile program of the reference
// (tmp/ir.mlir:89-157: S = Q.K^T per K tile, running row max, exp2 of the
// scaled scores, running row sum, acc_o rescale, acc_o += P.V, final
// division) and the softmax of benchmark/layout/execution/
// tail_attention_reference.py:81-114; the reference executes it only as a
// three-pass D64 kernel (tiled_attention.py:210-728).  Here it is one pass
// with an online softmax.
//
// Layout choices (all per 64-lane wave, MFMA v_mfma_f32_32x32x16):
//  * S^T = K.Q^T, not S = Q.K^T: the 32x32 accumulator keeps one column per
//    lane, so lane l owns query l%32 and holds 16 of its key scores per
//    32-key tile.  Row max / row sum of a query are in-lane reductions plus
//    one exchange with lane l^32.
//  * The S^T accumulator element r of lane (l32, h) is key 8(r/4)+4h+r%4.
//    Converted to bf16 it is used unchanged as the B operand (P^T) of
//    O^T = V^T.P^T: MFMA k-slot (h, e) then means key
//    16ks + (e < 4 ? 4h+e : 8+4h+e-4).  V stays row-major in LDS; its
//    V^T fragments, in exactly that key order, come from the gfx950
//    transposing LDS read ds_read_b64_tr_b16 (two per fragment).
//  * O^T accumulators also keep query = lane%32, so the softmax rescale is a
//    per-lane scalar.  Rescaling is lazy: the running max only moves when a
//    block's max exceeds it by more than 2^8 in the exp2 domain, keeping
//    every p <= 256 (exact in the final O / l, representable in bf16/f16).
//  * K and V tiles (64 keys x 2D bytes each) arrive by LDS-DMA with XOR
//    swizzles chosen for their read patterns, double-buffered: the loads of
//    key block j+1 are in flight during the MFMAs and softmax of block j.
//  * K stored [batch, heads, head_dim, seq] (KT; the layout of the
//    reference's FA tile program, tmp/ir.mlir:92) is staged as head_dim rows
//    of 64 keys and its fragments come from the same transposing LDS read
//    as V^T's, which delivers head_dim in the order (e < 4 ? 4h+e :
//    8+4h+e-4) per lane half h; the Q fragments are loaded in that order
//    too, so the products pair up and no transpose or copy of K is made.
//    Below head_dim 32 the V rows are padded to 32 dims in LDS (the DMA
//    writes zeros there), so O^T keeps its 32-row MFMA tile; the padded rows
//    are never stored.
//  * Key blocks that need no mask run in a loop without mask code; the few
//    blocks at the sequence end / causal diagonal run a masked copy.

#pragma once

#include "common.h"
#include "kernels.h"

namespace frisk {

namespace {

// Every building block of the kernel body is inlined: a lambda left as a
// call keeps its captures in private memory, and the buffer resources
// loaded from there are no longer known to be uniform.
#define FRISK_INLINE __attribute__((always_inline))

constexpr int kBN = 64;       // keys per block
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleSlack = 8.0f;  // log2 headroom before the running max moves

#define FRISK_WAIT_VMCNT0() __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8))
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <Elt T> struct AttnMfma;
template <> struct AttnMfma<Elt::BF16> {
  __device__ static inline f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack(float lo, float hi) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    v2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_bf16 with (1, 1)).
  __device__ static inline float dot2_ones(uint32_t w, float acc) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, w),
                                           __builtin_bit_cast(v2, 0x3f803f80u), acc, false);
  }
};
template <> struct AttnMfma<Elt::F16> {
  __device__ static inline f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack(float lo, float hi) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    v2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline float dot2_ones(uint32_t w, float acc) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, w), __builtin_bit_cast(v2, 0x3c003c00u),
                                  acc, false);
  }
};

// LDS geometry of one key block for head_dim D.
//  K: 64 rows of 2D bytes; chunk c of row r stored at c ^ swz_k(r), with
//     swz_k(r) = (r >> log2(16 / kc)) & (kc - 1) (kc = 2D / 16 chunks): the 16
//     rows one fragment read touches at one logical chunk land in 16
//     distinct 16-B bank groups.
//  V: 64 rows of 2 max(D, 32) bytes; the 4 rows (key & 3) of one transposed
//     read hit disjoint chunk pairs (swz_v).
template <int D> struct AttnGeom {
  static_assert(D == 16 || D == 32 || D == 64 || D == 128, "head_dim 16/32/64/128");
  static constexpr int kRB = 2 * D;                  // K row bytes
  static constexpr int kKC = kRB / 16;               // K chunks per row
  static constexpr int kKShift = D == 128 ? 0 : D == 64 ? 1 : D == 32 ? 2 : 3;
  static constexpr int kDP = D < 32 ? 32 : D;        // padded dims of V / O^T
  static constexpr int kRV = 2 * kDP;                // V row bytes
  static constexpr int kVC = kRV / 16;               // V chunks per row
  static constexpr int kKTile = kBN * kRB;
  static constexpr int kVTile = kBN * kRV;
  static constexpr int kBuf = kKTile + kVTile;
  static constexpr int kKSteps = D / 16;             // S^T MFMA k-steps
  static constexpr int kH1 = (kKSteps + 1) / 2;      // first half of them
  static constexpr int kH2 = kKSteps - kH1;
  static constexpr int kDT = kDP / 32;               // O^T tiles of 32 dims
  __device__ static int swz_k(int r) { return (r >> kKShift) & (kKC - 1); }
  // K^T rows (K stored head_dim-major): 64 keys = 8 chunks, read by the
  // transposing pattern of V^T at 8 chunks per row, so V's swizzle for
  // that width.
  __device__ static int swz_kt(int r) { return 2 * ((r >> 1) & 1); }
  __device__ static int swz_v(int r) {
    if constexpr (kVC == 16) return 4 * (r & 3);
    else if constexpr (kVC == 8) return 2 * ((r >> 1) & 1);
    else return 0;
  }
};

__device__ __forceinline__ float pair_reduce(float x, bool max_op) {
  // Combines lane l with lane l^32 without the LDS pipe: v_permlane32_swap
  // of x with itself leaves x[l % 32] in one result and x[l % 32 + 32] in
  // the other, on every lane (every attention parity test depends on it).  A
  // ds_bpermute here made the softmax wait, through the in-order LDS
  // counter, for the Vᵀ fragment reads issued before it.  max and + are
  // commutative, so every lane gets the bits the exchange gave before.
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float a = __builtin_bit_cast(float, (uint32_t)r[0]);
  const float b = __builtin_bit_cast(float, (uint32_t)r[1]);
  return max_op ? fmaxf(a, b) : a + b;
}

}  // namespace

// QT query tiles of 32 per wave, NW waves per workgroup:
// BM = 32 * QT * NW queries per workgroup.  OUT is T or F32.
template <Elt T, Elt OUT, int D, int QT, int NW, bool CAUSAL, bool KT = false>
__global__ __launch_bounds__(64 * NW) void attn_fwd_kernel(
    const char* __restrict__ Q, const char* __restrict__ K, const char* __restrict__ V,
    char* __restrict__ O, float* __restrict__ LSE, int heads, int seq_q, int seq_k,
    int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, int64_t o_ss,
    float scale_log2, int q_blocks) {
#if defined(__HIP_DEVICE_COMPILE__)
  using Mf = AttnMfma<T>;
  using G = AttnGeom<D>;
  constexpr int BM = 32 * QT * NW;
  extern __shared__ __attribute__((aligned(1024))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;

  // Block -> (batch*head, slot).  All slots of one head are kept on one
  // XCD (block ids congruent mod 8) so its K/V stay in one L2.  Without a
  // mask a slot is one query block.  Under a causal mask slot s runs query
  // block q_blocks-1-s and then query block s (the middle one alone when
  // q_blocks is odd): every workgroup visits about the same number of key
  // blocks, the heavy half first (b4 h32 s4096 d128 causal: +2-3%).
  const int slots = CAUSAL ? (q_blocks + 1) / 2 : q_blocks;
  int bh, slot;
  {
    const int pid = blockIdx.x;
    const int nbh = gridDim.x / slots;
    if (nbh % 8 == 0) {
      const int xcd = pid & 7, idx = pid >> 3;
      bh = (idx / slots) * 8 + xcd;
      slot = idx % slots;
    } else {
      bh = pid / slots;
      slot = pid % slots;
    }
  }
  const int n_qblocks = (CAUSAL && q_blocks - 1 - slot != slot) ? 2 : 1;
  for (int run = 0; run < n_qblocks; ++run) {
    const int qb = CAUSAL ? (run == 0 ? q_blocks - 1 - slot : slot) : slot;
    // The previous query block's last key block may still be read from LDS.
    if (run > 0) __syncthreads();
    const int b = bh / heads, h = bh % heads;
    const int q0 = qb * BM;
    const int diag = seq_k - seq_q;  // key j is visible to query i iff j <= i + diag
    int kv_len = seq_k;
    if (CAUSAL) kv_len = min(seq_k, q0 + BM + diag);
    const int nkb = kv_len > 0 ? (kv_len + kBN - 1) / kBN : 0;

    const char* qh = Q + (b * q_sb + h * q_sh) * 2;
    const char* kh = K + (b * k_sb + h * k_sh) * 2;
    const char* vh = V + (b * v_sb + h * v_sh) * 2;

    // ---- Q fragments (B operand of S^T = K.Q^T), loaded once -------------
    // Lane half h holds head_dim 16ds + 8h .. +7 of its query, or with KT
    // 16ds + 4h .. +3 and 16ds + 8 + 4h .. +3 (the order the transposing
    // read gives the K^T fragments).
    const int wq0 = q0 + wave * 32 * QT;  // first query of this wave
    i32x4 qf[QT][G::kKSteps];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int qi = min(wq0 + t * 32 + l32, seq_q - 1);
      const char* row = qh + (int64_t)qi * q_ss * 2;
#pragma unroll
      for (int ds = 0; ds < G::kKSteps; ++ds) {
        if constexpr (KT) {
          typedef int i32x2 __attribute__((ext_vector_type(2)));
          const i32x2 lo = *(const i32x2*)(row + ds * 32 + half * 8);
          const i32x2 hi = *(const i32x2*)(row + ds * 32 + 16 + half * 8);
          qf[t][ds] = i32x4{lo[0], lo[1], hi[0], hi[1]};
        } else {
          qf[t][ds] = *(const i32x4*)(row + ds * 32 + half * 16);
        }
      }
    }

    // ---- K and V tiles by LDS-DMA -------------------------------------------
    // One DMA instruction writes 1 KiB: lane L lands in row L / chunks-per-row,
    // physical chunk L % chunks-per-row, and fetches the logical chunk that
    // the row's swizzle puts there.  Rows past seq_k and the V padding dims
    // (head_dim < 32) read zeros (offsets past the buffer range).
    // With KT, k_ss is the stride between head_dim rows of K^T and keys
    // are contiguous: a row holds seq_k keys.
    const __amdgpu_buffer_rsrc_t rsk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)kh, (short)0,
        (int)min(KT ? (int64_t)(D - 1) * k_ss * 2 + (int64_t)seq_k * 2
                    : (int64_t)(seq_k - 1) * k_ss * 2 + D * 2,
                 (int64_t)0x7fffffff),
        0x00020000);
    const __amdgpu_buffer_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)vh, (short)0, (int)min((int64_t)(seq_k - 1) * v_ss * 2 + D * 2, (int64_t)0x7fffffff),
        0x00020000);
    constexpr int kKIns = G::kKTile / 1024, kVIns = G::kVTile / 1024;  // per tile
    constexpr int kKI = (kKIns + NW - 1) / NW, kVI = (kVIns + NW - 1) / NW;  // per wave
    uint32_t k_off[kKI], v_off[kVI];
    int k_row[kKI], v_row[kVI];
#pragma unroll
    for (int i = 0; i < kKI; ++i) {
      if constexpr (KT) {
        // Row r of the K^T tile: head_dim index r, 64 keys (8 chunks).
        const int r = (wave * kKI + i) * 8 + lane / 8;
        const int c = (lane % 8) ^ G::swz_kt(r);
        k_row[i] = (wave * kKI + i) < kKIns ? c * 8 : 1 << 30;  // first key of the chunk
        k_off[i] = (uint32_t)(r * k_ss * 2) + (c << 4);
      } else {
        const int r = (wave * kKI + i) * (1024 / G::kRB) + lane / G::kKC;
        const int c = (lane % G::kKC) ^ G::swz_k(r);
        k_row[i] = (wave * kKI + i) < kKIns ? r : 1 << 30;
        k_off[i] = (uint32_t)(r * k_ss * 2) + (c << 4);
      }
    }
#pragma unroll
    for (int i = 0; i < kVI; ++i) {
      const int r = (wave * kVI + i) * (1024 / G::kRV) + lane / G::kVC;
      const int c = (lane % G::kVC) ^ G::swz_v(r);
      v_row[i] = ((wave * kVI + i) < kVIns && c * 8 < D) ? r : 1 << 30;
      v_off[i] = (uint32_t)(r * v_ss * 2) + (c << 4);
    }
    auto issue_k = [&](int kb, char* dst) FRISK_INLINE {
      // A K block starts kBN keys further: kBN rows, or with KT kBN columns.
      const uint32_t kbase = (uint32_t)(KT ? (int64_t)kb * kBN * 2 : (int64_t)kb * kBN * k_ss * 2);
#pragma unroll
      for (int i = 0; i < kKI; ++i) {
        if ((wave * kKI + i) >= kKIns) continue;  // wave-uniform
        const int r = kb * kBN + k_row[i];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsk, (lds_ptr_t)(dst + (wave * kKI + i) * 1024), 16,
            r < seq_k ? kbase + k_off[i] : 0x80000000u, 0, 0, 0);
      }
    };
    auto issue_v = [&](int kb, char* dst) FRISK_INLINE {
      const uint32_t vbase = (uint32_t)((int64_t)kb * kBN * v_ss * 2);
#pragma unroll
      for (int i = 0; i < kVI; ++i) {
        if ((wave * kVI + i) >= kVIns) continue;  // wave-uniform
        const int r = kb * kBN + v_row[i];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsv, (lds_ptr_t)(dst + G::kKTile + (wave * kVI + i) * 1024), 16,
            r < seq_k ? vbase + v_off[i] : 0x80000000u, 0, 0, 0);
      }
    };
    auto issue_kv = [&](int kb, int buf) FRISK_INLINE {
      char* dst = smem + buf * G::kBuf;
      issue_k(kb, dst);
      issue_v(kb, dst);
    };

    // ---- V^T fragments by transposing LDS reads ------------------------------
    // ds_read_b64_tr_b16: inside each 16-lane group, lane j receives element
    // j%4 of the 8 B read by lanes j/4 + 4e, e = 0..3.  Lane 4e+q of group G
    // (h = G/2, dg = G%2) reads V[16kk + 4h + e (+8)][32dt + 16dg + 4q .. +3],
    // so lane l receives V[16kk + 4h + 0..3 (+8)][32dt + l%32]: the A operand
    // of O^T = V^T.P^T with k-slots (h, e) -> key 16kk + (e < 4 ? 4h+e :
    // 8+4h+e-4), the key order of P taken from the S^T accumulators.
    int vt_off[G::kDT];
    {
      const int g = lane >> 4, hh = g >> 1, dg = g & 1, e = (lane >> 2) & 3, q = lane & 3;
#pragma unroll
      for (int dt = 0; dt < G::kDT; ++dt) {
        // The row is 16kk + 4hh + e (+8): its swizzle only depends on e.
        const int chunk = (4 * dt + 2 * dg + (q >> 1)) ^ G::swz_v(4 * hh + e);
        vt_off[dt] = G::kKTile + (4 * hh + e) * G::kRV + (chunk << 4) + 8 * (q & 1);
      }
    }

    // K^T fragments (KT) by the same transposing read: lane 4e+q of group G
    // (h = G/2, kg = G%2) reads K^T[16ds + 4h + e (+8)][32kt + 16kg + 4q ..
    // +3], so lane l receives head_dim 16ds + 4h + 0..3 (+8) of key
    // 32kt + l%32: the A operand of S^T = K.Q^T in the head_dim order of
    // the Q fragments above.
    int kt_off[2];
    if constexpr (KT) {
      const int g = lane >> 4, hh = g >> 1, kg = g & 1, e = (lane >> 2) & 3, q = lane & 3;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int chunk = (4 * kt + 2 * kg + (q >> 1)) ^ G::swz_kt(4 * hh + e);
        kt_off[kt] = (4 * hh + e) * 128 + (chunk << 4) + 8 * (q & 1);
      }
    }

    // ---- state ---------------------------------------------------------------
    f32x16 o[QT][G::kDT];
    float m[QT], l[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      m[t] = -__builtin_inff();
      l[t] = 0.0f;
#pragma unroll
      for (int dt = 0; dt < G::kDT; ++dt) o[t][dt] = f32x16{};
    }

    // ---- building blocks ----------------------------------------------------
    // K fragments of head-dim steps h0 .. h0+n-1 for both 32-key tiles.
    auto read_k = [&](const char* ks, int h0, auto& kf) FRISK_INLINE {
      constexpr int n = sizeof(kf[0]) / sizeof(kf[0][0]);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int r = kt * 32 + l32;
#pragma unroll
        for (int i = 0; i < n; ++i) {
          if constexpr (KT) {
            const char* p = ks + kt_off[kt] + (h0 + i) * 16 * 128;
            const s16x4 lo = lds_read_tr16(p);
            const s16x4 hi = lds_read_tr16(p + 8 * 128);
            typedef int i32x2 __attribute__((ext_vector_type(2)));
            const i32x2 a = __builtin_bit_cast(i32x2, lo), b = __builtin_bit_cast(i32x2, hi);
            kf[kt][i] = i32x4{a[0], a[1], b[0], b[1]};
          } else {
            kf[kt][i] =
                *(const i32x4*)(ks + r * G::kRB + (((2 * (h0 + i) + half) ^ G::swz_k(r)) << 4));
          }
        }
      }
    };
    // V^T fragments of key steps k0, k0+1 (16 keys each).
    auto read_v = [&](const char* ks, int k0, i32x4 (&vf)[2][G::kDT]) FRISK_INLINE {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int dt = 0; dt < G::kDT; ++dt) {
          const char* p = ks + vt_off[dt] + (k0 + i) * 16 * G::kRV;
          // Through the restrict-pointer helper: a bare intrinsic here
          // waited for the next block's K/V DMA (vmcnt(0)) before the first
          // read (C5 non-causal 1063 -> 1098 TFLOP/s without that wait).
          const s16x4 lo = lds_read_tr16(p);
          const s16x4 hi = lds_read_tr16(p + 8 * G::kRV);
          typedef int i32x2 __attribute__((ext_vector_type(2)));
          const i32x2 a = __builtin_bit_cast(i32x2, lo), b = __builtin_bit_cast(i32x2, hi);
          vf[i][dt] = i32x4{a[0], a[1], b[0], b[1]};
        }
    };
    // Online softmax of one key block in the exp2 domain:
    // p = exp2(s * scale_log2 - m).  The max is taken on raw scores
    // (scale_log2 > 0 commutes with max).  Masked blocks (the sequence tail,
    // and blocks crossing this wave's causal diagonal) apply the key mask.
    auto softmax = [&](f32x16 (&s)[QT][2], i32x4 (&pf)[QT][4], int kbase, auto masked_tag) FRISK_INLINE {
      constexpr bool kMasked = decltype(masked_tag)::value;
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        if constexpr (kMasked) {
          const int qi = wq0 + t * 32 + l32;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = kbase + kt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
              if (key >= seq_k || (CAUSAL && key > qi + diag)) s[t][kt][r] = -__builtin_inff();
            }
        }
        float mraw = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) mraw = fmaxf(mraw, s[t][kt][r]);
        const float mb = pair_reduce(mraw, true) * scale_log2;
        const bool move = mb > m[t] + kRescaleSlack;
        if (__builtin_amdgcn_ballot_w64(move)) {
          // exp2(-inf) = 0 on a row's first visible block; rows that do not
          // move keep alpha = 1 (m - mn would be NaN for m = mn = -inf).
          const float alpha = move ? __builtin_amdgcn_exp2f(m[t] - mb) : 1.0f;
          m[t] = move ? mb : m[t];
          l[t] *= alpha;
#pragma unroll
          for (int dt = 0; dt < G::kDT; ++dt) o[t][dt] *= alpha;
        }
        // A row with every key masked so far keeps m = -inf; subtracting 0
        // instead gives its (all -inf) scores p = 0 rather than NaN.
        const float nm = m[t] == -__builtin_inff() ? 0.0f : -m[t];
        float rs = l[t];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int kt = kk >> 1, r0 = 8 * (kk & 1);
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][kt][r0 + 2 * e], scale_log2, nm));
            const float p1 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][kt][r0 + 2 * e + 1], scale_log2, nm));
            w[e] = Mf::pack(p0, p1);
            rs = Mf::dot2_ones(w[e], rs);  // the row sum uses the rounded P of the PV product
          }
          pf[t][kk] = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
        l[t] = rs;
      }
    };

    // Key blocks [0, n_plain) need no mask for any wave of this workgroup
    // (they end at or before wave 0's causal diagonal and the sequence end);
    // the remaining few run the masked variant.
    int n_plain = seq_k / kBN;
    if (CAUSAL) n_plain = min(n_plain, max(0, (q0 + diag + 1) / kBN));
    n_plain = min(n_plain, nkb);

    if (nkb > 0) {
      issue_kv(0, 0);
      FRISK_WAIT_VMCNT0();
      __syncthreads();
    }
    // Drain the scalar loads of kernel arguments used after the loop: with
    // them pending at loop entry the LGKM counter is unordered and every LDS
    // read in the loop would be waited for with lgkmcnt(0).
    __builtin_amdgcn_s_waitcnt(0xC07F);

    // One key block: S^T = K.Q^T, online softmax, O^T += V^T.P^T.  S^T runs
    // in two halves of the head-dim steps: the K fragments of a half are
    // read together (one LDS latency per half, not per MFMA) and the second
    // half's reads issue under the first half's MFMAs.  The first half of
    // the V^T fragments is read before the softmax, whose VALU work hides
    // it.
    auto key_block = [&](const char* ks, int kbase, auto masked_tag, auto&& dma) FRISK_INLINE {
      // Under a causal mask a block that starts past the last key this
      // wave's queries see gives p = 0 in every row: the wave skips its
      // arithmetic (still taking part in the loads and barriers); its state
      // is unchanged, as the masked arithmetic would leave it.
      if constexpr (CAUSAL && decltype(masked_tag)::value)
        if (kbase > wq0 + 32 * QT - 1 + diag) {
          dma();  // this wave's share of the next block's loads
          return;
        }
      f32x16 s[QT][2];
#pragma unroll
      for (int t = 0; t < QT; ++t) s[t][0] = s[t][1] = f32x16{};
      i32x4 kf0[2][G::kH1], kf1[2][G::kH2 > 0 ? G::kH2 : 1];
      read_k(ks, 0, kf0);
      __builtin_amdgcn_sched_barrier(0);
      // The next block's loads (dma) go out behind the first fragment
      // reads, whose latency they fill.
      dma();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (G::kH2 > 0) read_k(ks, G::kH1, kf1);
#pragma unroll
      for (int i = 0; i < G::kH1; ++i)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int t = 0; t < QT; ++t) s[t][kt] = Mf::run(kf0[kt][i], qf[t][i], s[t][kt]);
      __builtin_amdgcn_sched_barrier(0);
      i32x4 vf0[2][G::kDT], vf1[2][G::kDT];
      read_v(ks, 0, vf0);
      if constexpr (G::kH2 > 0) {
#pragma unroll
        for (int i = 0; i < G::kH2; ++i)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int t = 0; t < QT; ++t)
              s[t][kt] = Mf::run(kf1[kt][i], qf[t][G::kH1 + i], s[t][kt]);
      }
      // The second half of the V^T fragments, read here once the K
      // fragments are dead, so that the softmax hides its latency as well
      // (C5 non-causal 1097 -> 1128 TFLOP/s; causal, with the 8-wave
      // workgroups, 944 -> 979-989).
      read_v(ks, 2, vf1);
      __builtin_amdgcn_sched_barrier(0);
      i32x4 pf[QT][4];
      softmax(s, pf, kbase, masked_tag);
      // O^T += V^T . P^T over 4 key steps of 16.
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int dt = 0; dt < G::kDT; ++dt)
#pragma unroll
          for (int t = 0; t < QT; ++t) o[t][dt] = Mf::run(vf0[i][dt], pf[t][i], o[t][dt]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int dt = 0; dt < G::kDT; ++dt)
#pragma unroll
          for (int t = 0; t < QT; ++t) o[t][dt] = Mf::run(vf1[i][dt], pf[t][2 + i], o[t][dt]);
    };

    // Block j uses buffer j & 1.  In the unmasked blocks of 8-wave
    // workgroups without a causal mask that is a compile-time constant (two
    // steps per trip), so the fragment reads add the buffer base as an
    // immediate offset to block-invariant lane addresses instead of a VALU
    // add per read (C5 non-causal +2.9-3.6%, bit-identical).  The masked
    // blocks, the causal kernels (no gain measured, 256 VGPRs) and the
    // 4-wave kernels (-17%) keep one copy of the step: the second copy's
    // hoisted addresses cost registers they do not have.
    auto step = [&](int j, auto masked_tag, auto bufc) FRISK_INLINE {
      const int buf = decltype(bufc)::value < 0 ? (j & 1) : decltype(bufc)::value;
      const bool more = j + 1 < nkb;
      // Without a causal mask the next block's loads go out behind this
      // block's first K fragment reads; the causal kernels, at their
      // register limit (spills), issue them first.
      if constexpr (CAUSAL) {
        if (more) issue_kv(j + 1, buf ^ 1);
        key_block(smem + buf * G::kBuf, j * kBN, masked_tag, []() FRISK_INLINE {});
      } else {
        key_block(smem + buf * G::kBuf, j * kBN, masked_tag, [&]() FRISK_INLINE {
          if (more) issue_kv(j + 1, buf ^ 1);
        });
      }
      if (more) FRISK_WAIT_VMCNT0();
      __syncthreads();
    };
    using BufRt = std::integral_constant<int, -1>;
    using Buf0 = std::integral_constant<int, 0>;
    using Buf1 = std::integral_constant<int, 1>;
    int j = 0;
    if constexpr (NW == 8 && !CAUSAL) {
      for (; j + 1 < n_plain; j += 2) {
        step(j, std::false_type{}, Buf0{});
        step(j + 1, std::false_type{}, Buf1{});
      }
    }
    for (; j < n_plain; ++j) step(j, std::false_type{}, BufRt{});
    for (; j < nkb; ++j) step(j, std::true_type{}, BufRt{});

    // ---- epilogue: O = O^T / l, LSE -----------------------------------------
    constexpr int kOB = EltInfo<OUT>::bytes;
    char* oh = O + (b * o_sb + h * o_sh) * kOB;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const float lt = pair_reduce(l[t], false);  // both lane halves of the row
      const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
      const int qi = wq0 + t * 32 + l32;
      if (qi < seq_q) {
        char* row = oh + (int64_t)qi * o_ss * kOB;
#pragma unroll
        for (int dt = 0; dt < G::kDT; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d = dt * 32 + 8 * g + 4 * half;
            if (d >= D) continue;  // V padding dims (head_dim < 32)
            if constexpr (OUT == Elt::F32) {
              *(f32x4*)(row + d * 4) = f32x4{o[t][dt][4 * g + 0] * inv, o[t][dt][4 * g + 1] * inv,
                                             o[t][dt][4 * g + 2] * inv, o[t][dt][4 * g + 3] * inv};
            } else {
              typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
              const u32x2 w = {Mf::pack(o[t][dt][4 * g + 0] * inv, o[t][dt][4 * g + 1] * inv),
                               Mf::pack(o[t][dt][4 * g + 2] * inv, o[t][dt][4 * g + 3] * inv)};
              *(u32x2*)(row + d * 2) = w;
            }
          }
        if (LSE && half == 0)
          LSE[(int64_t)bh * seq_q + qi] =
              lt > 0.0f ? (m[t] + __log2f(lt)) * kLn2 : -__builtin_inff();
      }
    }
  }  // query blocks of this slot
#endif  // __HIP_DEVICE_COMPILE__
}

// One workgroup shape: NW waves x 32 queries.
template <Elt T, Elt OUT, int D, int NW, bool CAUSAL, bool KT>
static hipError_t launch_attn_nw(const AttnArgs& a, hipStream_t stream) {
  constexpr int QT = 1, BM = 32 * QT * NW;
  auto kern = attn_fwd_kernel<T, OUT, D, QT, NW, CAUSAL, KT>;
  constexpr int lds = 2 * AttnGeom<D>::kBuf;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (attr != hipSuccess) return attr;
  const int q_blocks = (int)((a.seq_q + BM - 1) / BM);
  const int64_t slots = CAUSAL ? (q_blocks + 1) / 2 : q_blocks;
  const int64_t blocks = slots * a.batch * a.heads;
  const float scale_log2 = a.sm_scale * kLog2e;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * NW), lds, stream, (const char*)a.q,
                     (const char*)a.k, (const char*)a.v, (char*)a.o, a.lse, (int)a.heads,
                     (int)a.seq_q, (int)a.seq_k, a.q_sb, a.q_sh, a.q_ss, a.k_sb, a.k_sh, a.k_ss,
                     a.v_sb, a.v_sh, a.v_ss, a.o_sb, a.o_sh, a.o_ss, scale_log2, q_blocks);
  return hipGetLastError();
}

// Workgroup shape per launch: a.waves when the request names one, else
// plan::attn_waves (launch_plan.h, which holds the measurements behind the
// rule).  Head_dim 64 and below run 4-wave workgroups only.  Every query's
// arithmetic is the same in both shapes (same key blocks in the same order;
// a masked block with no hidden key computes what an unmasked one does), so
// the choice never changes a result bit.
template <Elt T, Elt OUT, int D, bool CAUSAL, bool KT>
static hipError_t launch_attn_kt(const AttnArgs& a, hipStream_t stream) {
  if constexpr (D <= 64) {
    return launch_attn_nw<T, OUT, D, 4, CAUSAL, KT>(a, stream);
  } else {
    const int waves = a.waves ? a.waves
                              : plan::attn_waves(a.batch * a.heads, a.seq_q, D, CAUSAL, device_cus());
    return waves == 4 ? launch_attn_nw<T, OUT, D, 4, CAUSAL, KT>(a, stream)
                      : launch_attn_nw<T, OUT, D, 8, CAUSAL, KT>(a, stream);
  }
}

// K stored [.., seq, head_dim] or [.., head_dim, seq] (a.k_dmajor).
template <Elt T, Elt OUT, int D, bool CAUSAL>
static hipError_t launch_attn(const AttnArgs& a, hipStream_t stream) {
  return a.k_dmajor ? launch_attn_kt<T, OUT, D, CAUSAL, true>(a, stream)
                    : launch_attn_kt<T, OUT, D, CAUSAL, false>(a, stream);
}

// Every (input dtype, output dtype, mask) variant of one head_dim.
template <int D>
hipError_t attn_fwd_dispatch(const AttnArgs& a, hipStream_t s) {
  const bool f32_out = a.out == Elt::F32;
  if (a.dtype == Elt::BF16) {
    if (f32_out)
      return a.causal ? launch_attn<Elt::BF16, Elt::F32, D, true>(a, s)
                      : launch_attn<Elt::BF16, Elt::F32, D, false>(a, s);
    return a.causal ? launch_attn<Elt::BF16, Elt::BF16, D, true>(a, s)
                    : launch_attn<Elt::BF16, Elt::BF16, D, false>(a, s);
  }
  if (a.dtype == Elt::F16) {
    if (f32_out)
      return a.causal ? launch_attn<Elt::F16, Elt::F32, D, true>(a, s)
                      : launch_attn<Elt::F16, Elt::F32, D, false>(a, s);
    return a.causal ? launch_attn<Elt::F16, Elt::F16, D, true>(a, s)
                    : launch_attn<Elt::F16, Elt::F16, D, false>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace frisk
