// indexer_tile.h -- one wave's lightning-indexer tile on MFMA (gfx950).
//
//   I[t,s] = sum_j w[t,j] * ReLU(<q[t,j,:], k[s,:]>)      (lightning_indexer.py:26-33)
//
// A wave owns 4 consecutive queries t0..t0+3 and walks the keys in blocks of
// 16.  The GEMM rows are (query, head) pairs, 4 queries x 4 heads = 16 rows
// per MFMA, one MFMA row-group per group of 4 heads ("head group", hg).  With
// that row order the 16x16 MFMA output layout puts all 4 heads of one
// (query, key) pair in the 4 accumulator registers of one lane:
//     lane l  ->  query t0 + l/16, key s0 + l%16, heads 4hg..4hg+3
// so the ReLU * w head reduction is 4 v_max + 4 v_fma per lane per head
// group, entirely in registers -- no shuffles, no LDS.
//
// The reduction dimension DI is permuted so every lane's operand slice is
// contiguous in memory: lane group g = l/16 owns dims [g*DI/4, (g+1)*DI/4),
// and MFMA step kk consumes element kk (fp32, K=4 per MFMA) or elements
// 8kk..8kk+7 (bf16/fp16, K=32 per MFMA) of that slice.  A and B use the same
// permutation, so the sum over DI is unchanged and each lane loads its slice
// with 16-byte vector loads.
//
//   fp32 inputs : v_mfma_f32_16x16x4_f32     (exact fp32 products, fp32 sum)
//   bf16 inputs : v_mfma_f32_16x16x32_bf16   (exact products, fp32 sum)
//   fp16 inputs : v_mfma_f32_16x16x32_f16
#pragma once

#include "dsa_device.h"

namespace dsa {

// Per-lane operand slice of DI/4 elements in MFMA-ready registers.
template <typename Tag, int E>
struct Slice;

template <int E>
struct Slice<F32, E> {
  static constexpr int kSteps = E;  // one MFMA per element
  float v[E];
  __device__ __forceinline__ void load(const float* __restrict__ p) { load_f32<E>(p, v); }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < E; ++i) v[i] = 0.f;
  }
  __device__ __forceinline__ f32x4 mfma(int i, const Slice& b, f32x4 acc) const {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(v[i], b.v[i], acc, 0, 0, 0);
  }
};

template <typename Tag, int E>
struct Slice16 {
  static_assert(E % 8 == 0, "16-bit slices are whole 8-element MFMA operands");
  static constexpr int kSteps = E / 8;
  uint4 v[E / 8];
  __device__ __forceinline__ void load(const uint16_t* __restrict__ p) {
#pragma unroll
    for (int i = 0; i < E / 8; ++i) v[i] = *reinterpret_cast<const uint4*>(p + 8 * i);
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < E / 8; ++i) v[i] = make_uint4(0u, 0u, 0u, 0u);
  }
};

template <int E>
struct Slice<BF16, E> : Slice16<BF16, E> {
  __device__ __forceinline__ f32x4 mfma(int i, const Slice& b, f32x4 acc) const {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, this->v[i]),
                                                   __builtin_bit_cast(bf16x8, b.v[i]), acc, 0,
                                                   0, 0);
  }
};

template <int E>
struct Slice<F16, E> : Slice16<F16, E> {
  __device__ __forceinline__ f32x4 mfma(int i, const Slice& b, f32x4 acc) const {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, this->v[i]),
                                                  __builtin_bit_cast(f16x8, b.v[i]), acc, 0, 0,
                                                  0);
  }
};

// fp8 slices: E bytes as 16-byte chunks; the MFMA (16x16x128) takes two
// chunks of A and of B per step (indexer.hip).
template <int E>
struct Slice<FP8, E> {
  static_assert(E % 16 == 0, "fp8 slices are whole 16-byte chunks");
  uint4 v[E / 16];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ p) {
#pragma unroll
    for (int i = 0; i < E / 16; ++i) v[i] = *reinterpret_cast<const uint4*>(p + 16 * i);
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < E / 16; ++i) v[i] = make_uint4(0u, 0u, 0u, 0u);
  }
};

// Computes scores of queries t0..t0+4*QG-1 (batch row base pointers given)
// against keys [s_begin, s_end) in super-blocks of 16*KB keys and hands each
// finished super-block to sink(s0, sc) where lane l holds sc[qg][kb] = score
// of query t0 + 4*qg + l/16 and key s0 + 16*kb + l%16 (for QG = 1, sc[kb]).
// Entries with key > query, key >= T or query >= T hold garbage/-inf; the
// sink applies the causal mask and bounds.  QG query groups of 4 share every
// key block a wave loads, so QG = 2 halves the key loads per query.
//
// q : [T, HI, DI] of this batch element   k : [T, DI]   w : [T, HI], rows of
// consecutive tokens ldq / ldk / ldw elements apart.
template <typename Tag, int DI, int KB, int QG = 1, typename Sink>
__device__ __forceinline__ void indexer_rows(const typename Tag::raw* __restrict__ q,
                                             const typename Tag::raw* __restrict__ k,
                                             const typename Tag::raw* __restrict__ w, int T,
                                             int HI, int64_t ldq, int64_t ldk, int64_t ldw,
                                             int t0, int s_begin, int s_end, Sink&& sink) {
  constexpr int E = DI / 4;
  using S = Slice<Tag, E>;
  const int lane = lane_id();
  const int g = lane >> 4;   // lane group: reduction slice; output query
  const int r16 = lane & 15; // A row / B column
  const int nhg = (HI + 3) >> 2;

  // A row of this lane in query group qg: query t0 + 4qg + r16/4, head
  // 4*hg + r16%4; output query t0 + 4qg + g.
  const int ha = r16 & 3;

  auto load_a = [&](int qg, int hg, S& a, float (&wv)[4]) {
    const int qa = t0 + 4 * qg + (r16 >> 2);
    const int qo = t0 + 4 * qg + g;
    const int head = 4 * hg + ha;
    if (qa < T && head < HI)
      a.load(q + static_cast<int64_t>(qa) * ldq + head * DI + g * E);
    else
      a.zero();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hw = 4 * hg + r;
      wv[r] = (qo < T && hw < HI) ? to_f32(Tag{}, w[static_cast<int64_t>(qo) * ldw + hw]) : 0.f;
    }
  };
  // Head-group-invariant operands when HI <= 4: load once.
  S a_cached[QG];
  float w_cached[QG][4];
  if (nhg == 1) {
#pragma unroll
    for (int qg = 0; qg < QG; ++qg) load_a(qg, 0, a_cached[qg], w_cached[qg]);
  }

  // Key blocks of super-block s0 -> registers.  The next super-block is
  // loaded while the MFMAs of the current one run.
  auto load_b = [&](int s0, S (&bk)[KB]) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int s = s0 + 16 * kb + r16;
      if (s < T)
        bk[kb].load(k + static_cast<int64_t>(s) * ldk + g * E);
      else
        bk[kb].zero();
    }
  };
  S bk[KB];
  load_b(s_begin, bk);
  for (int s0 = s_begin; s0 < s_end; s0 += 16 * KB) {
    S bn[KB];
    if (s0 + 16 * KB < s_end) load_b(s0 + 16 * KB, bn);
    float sc[QG][KB];
#pragma unroll
    for (int qg = 0; qg < QG; ++qg)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sc[qg][kb] = 0.f;

    for (int hg = 0; hg < nhg; ++hg) {
#pragma unroll
      for (int qg = 0; qg < QG; ++qg) {
        S a;
        float wv[4];
        if (nhg == 1) {
          a = a_cached[qg];
#pragma unroll
          for (int r = 0; r < 4; ++r) wv[r] = w_cached[qg][r];
        } else {
          load_a(qg, hg, a, wv);
        }
        f32x4 acc[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        // the unit's MFMAs at raised wave priority, its epilogue at the normal
        // one: the SIMD's other waves' VALU work fills in behind the MFMAs
        // (fused kernel, config 1: 25.38 -> 25.22 us)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < S::kSteps; ++i) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) acc[kb] = a.mfma(i, bk[kb], acc[kb]);
        }
        __builtin_amdgcn_s_setprio(0);
        // ReLU on the bit pattern (one integer max; fmaxf on an MFMA result
        // takes a canonicalising max first): config 1 25.18 -> 24.95 us
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sc[qg][kb] = fmaf(wv[r], relu_f32(acc[kb][r]), sc[qg][kb]);
        }
      }
    }
    if constexpr (QG == 1) sink(s0, sc[0]);
    else sink(s0, sc);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) bk[kb] = bn[kb];
  }
}

}  // namespace dsa
