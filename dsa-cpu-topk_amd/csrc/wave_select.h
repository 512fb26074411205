// wave_select.h -- k-th largest of one LDS-resident score row, one wave.
// (wave_select_kth_bins, at the end, is the usual entry; wave_select_kth is
// its exact fallback.)
//
// Replaces the fused reference kernel's tl.sort(...)[TOP_K-1]
// (dsa_attention.py:151-155): same value (the k-th largest counting ties)
// without sorting.  Four MSD radix passes over 8-bit digits of the
// order-preserving key; each pass is a 256-bin LDS histogram built with
// ds_add by the wave, then a wave suffix-scan over the bins (4 per lane)
// finds the digit holding the k-th key.  A digit that holds a single key ends
// the search early.  The row is re-read from LDS on every pass, so no
// register array scales with T.
#pragma once

#include "dsa_device.h"

namespace dsa {

// row: n (>= k >= 1) valid scores in LDS, 16-byte aligned.  hist: 256 words
// of LDS private to this wave.  Returns the k-th largest value.
__device__ __forceinline__ float wave_select_kth(const float* row, int n, int k,
                                                 uint32_t* hist) {
  const int lane = lane_id();
  uint32_t prefix = 0;
  uint32_t krem = static_cast<uint32_t>(k);
  for (int p = 0; p < 4; ++p) {
    const int shift = 24 - 8 * p;
    reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    for (int s = 4 * lane; s < n; s += 4 * kWave) {
      const float4 f = *reinterpret_cast<const float4*>(row + s);
      const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t kk = float_to_key(fv[c]);
        const bool in = (s + c < n) && (p == 0 || (kk >> (shift + 8)) == prefix);
        if (in) atomicAdd(&hist[(kk >> shift) & 255u], 1u);
      }
    }
    wave_lds_sync();
    const uint4 h4 = reinterpret_cast<const uint4*>(hist)[lane];
    const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
    const uint32_t local = h[0] + h[1] + h[2] + h[3];
    const uint32_t incl = wave_inclusive_sum(local);
    const uint32_t total = wave_read_lane(incl, kWave - 1);
    const uint32_t above = total - incl;  // keys in higher lanes' bins
    const bool mine = above < krem && above + local >= krem;
    uint32_t bucket = 0, knew = 0, cnt = 0;
    if (mine) {
      uint32_t cum = above;
#pragma unroll
      for (int i = 3; i >= 0; --i) {
        if (cnt == 0u && cum + h[i] >= krem) {
          bucket = 4u * lane + i;
          knew = krem - cum;
          cnt = h[i];
        }
        cum += h[i];
      }
    }
    const uint64_t who = __ballot(mine);
    const int src = __ffsll(static_cast<unsigned long long>(who)) - 1;  // uniform
    bucket = wave_read_lane(bucket, src);
    knew = wave_read_lane(knew, src);
    cnt = wave_read_lane(cnt, src);
    prefix = (prefix << 8) | bucket;
    krem = knew;
    wave_lds_sync();  // histogram reads done before the next pass clears it
    if (p < 3 && cnt == 1u) {
      // The digit holds one key; fetch it.
      uint32_t hit = 0;
      for (int s = 4 * lane; s < n; s += 4 * kWave) {
        const float4 f = *reinterpret_cast<const float4*>(row + s);
        const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t kk = float_to_key(fv[c]);
          if ((s + c < n) && (kk >> shift) == prefix) hit = kk;
        }
      }
      const uint64_t m = __ballot(hit != 0u);
      return key_to_float(wave_read_lane(hit, __ffsll(static_cast<unsigned long long>(m)) - 1));
    }
  }
  return key_to_float(prefix);
}

// Same contract, usually in three reads of the row instead of four or more:
// the row's min and max, a 256-bin histogram linear in value between them
// (bins follow the data's density, so its ds_adds rarely collide), then the
// few values of the bin holding the k-th largest are gathered into `gl` (64
// words of wave-private LDS) and ranked against each other in registers:
// the wanted one has fewer than k' greater and at least k' greater or equal.
// Rows with a non-finite value, and bins holding more than 64 values (heavy
// ties), take wave_select_kth.  -0 is reported as +0, as the key order does.
// With the row's minimum lo, maximum hi and whether it holds a non-finite
// value (bad) already known (wave-uniform).
__device__ __forceinline__ float wave_select_kth_bins(const float* row, int n, int k,
                                                      uint32_t* hist, uint32_t* gl, float lo,
                                                      float hi, bool bad) {
  const int lane = lane_id();
  if (bad) return wave_select_kth(row, n, k, hist);
  if (!(hi > lo)) return hi + 0.0f;  // one value
  const float scale = 256.0f / (hi - lo);
  if (!(scale <= __FLT_MAX__)) return wave_select_kth(row, n, k, hist);
  reinterpret_cast<uint4*>(hist)[lane] = make_uint4(0u, 0u, 0u, 0u);
  wave_lds_sync();
  for (int s = 4 * lane; s < n; s += 4 * kWave) {
    const float4 f = *reinterpret_cast<const float4*>(row + s);
    const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (s + c < n) atomicAdd(&hist[value_bin(fv[c], lo, scale, 255.0f)], 1u);
  }
  wave_lds_sync();
  const uint32_t krem = static_cast<uint32_t>(k);
  const uint4 h4 = reinterpret_cast<const uint4*>(hist)[lane];
  const uint32_t h[4] = {h4.x, h4.y, h4.z, h4.w};
  const uint32_t local = h[0] + h[1] + h[2] + h[3];
  const uint32_t incl = wave_inclusive_sum(local);
  const uint32_t abv = wave_read_lane(incl, kWave - 1) - incl;  // values in higher lanes' bins
  const bool here = abv < krem && abv + local >= krem;
  uint32_t bsel = 0, brank = 0, bcnt = 0;
  if (here) {
    uint32_t cum = abv;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
      if (bcnt == 0u && cum + h[i] >= krem) {
        bsel = 4u * lane + i;
        brank = krem - cum;
        bcnt = h[i];
      }
      cum += h[i];
    }
  }
  const int src = __ffsll(static_cast<unsigned long long>(ballot(here))) - 1;
  bsel = wave_read_lane(bsel, src);
  brank = wave_read_lane(brank, src);
  bcnt = wave_read_lane(bcnt, src);
  wave_lds_sync();  // histogram reads done (the fallback clears it)
  if (bcnt > static_cast<uint32_t>(kWave)) return wave_select_kth(row, n, k, hist);
  uint32_t ng = 0;
  for (int s = 4 * lane; s < n; s += 4 * kWave) {
    const float4 f = *reinterpret_cast<const float4*>(row + s);
    const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool in = s + c < n && value_bin(fv[c], lo, scale, 255.0f) == static_cast<int>(bsel);
      const uint64_t m = ballot(in);
      if (in) gl[ng + lanes_below(m)] = __float_as_uint(fv[c]);
      ng += popc64(m);
    }
  }
  wave_lds_sync();
  const float mv = lane < static_cast<int>(bcnt) ? __uint_as_float(gl[lane]) : 0.0f;
  uint32_t gt = 0, ge = 0;
  for (uint32_t j = 0; j < bcnt; ++j) {
    const float o = __int_as_float(wave_read_lane(__float_as_int(mv), static_cast<int>(j)));  // no LDS read
    gt += (o > mv) ? 1u : 0u;
    ge += (o >= mv) ? 1u : 0u;
  }
  const bool hit = lane < static_cast<int>(bcnt) && gt < brank && ge >= brank;
  const float res = __int_as_float(
      wave_read_lane(__float_as_int(mv), __ffsll(static_cast<unsigned long long>(ballot(hit))) - 1));
  wave_lds_sync();  // gather-list reads done before the caller reuses it
  return res + 0.0f;
}

__device__ __forceinline__ float wave_select_kth_bins(const float* row, int n, int k,
                                                      uint32_t* hist, uint32_t* gl) {
  const int lane = lane_id();
  float lo = __builtin_huge_valf(), hi = -__builtin_huge_valf();
  bool bad = false;
  for (int s = 4 * lane; s < n; s += 4 * kWave) {
    const float4 f = *reinterpret_cast<const float4*>(row + s);
    const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (s + c < n) {
        lo = fminf(lo, fv[c]);
        hi = fmaxf(hi, fv[c]);
        bad = bad || !(fabsf(fv[c]) <= __FLT_MAX__);
      }
    }
  }
  return wave_select_kth_bins(row, n, k, hist, gl, wave_extreme_f32<false>(lo),
                              wave_extreme_f32<true>(hi), ballot(bad) != 0u);
}

}  // namespace dsa
