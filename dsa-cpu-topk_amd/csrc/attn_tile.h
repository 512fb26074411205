// attn_tile.h -- one wave computes sparse attention for one query (gfx950).
//
//   sel(s)   = s <= t  &&  score[s] >= thr                (dsa_attention.py:45-46, :258)
//   O[h,:]   = sum_{s in sel} softmax_s(<Q[t,h],K[s,h]> * scale) * V[s,h,:]
//
// The wave scans the score row 512 entries at a time (two float4 per lane),
// compacts the selected key positions in index order into a per-wave LDS
// list (ballot-free: a wave prefix sum of per-lane counts), then gathers
// only those K/V rows.  Each K (or V) row is HQ*D contiguous elements; lane
// l owns elements [l*EK, (l+1)*EK) -- one 16-byte-granular contiguous slice,
// so a row gather is a single coalesced wave load.  Per-head logits are a
// butterfly over the DQ/EK lanes of the head, or, when a head spans exactly
// as many lanes as a gather group has keys, a reduce-scatter that leaves one
// key's logit per lane (half_a_rs).  fp32 rows of 128 elements (8 bytes of a
// key per lane) take attend_query_pair instead: each half-wave reads one
// key's row, 16 bytes per lane, two keys per load.  Softmax is online (running
// max m, normaliser l) in the log2 domain with fp32 state, so the whole
// selected set is never materialised and any selected count works -- ties at
// the threshold can select more than k keys (the reference keeps ties).
#pragma once

#include <type_traits>
#include <utility>

#include "dsa_device.h"

namespace dsa {

constexpr int kListCap = 512;  // one 512-entry segment of the score row

// The keys s0 .. min(s0 + kListCap, t + 1) - 1 whose score is >= thr (a NaN
// score or threshold selects nothing), in index order, into `list`; returns
// how many (wave-uniform).  Lane l scans entries s0 + 8l .. s0 + 8l + 7 (two
// float4 through load4) and the lanes' counts are placed by a wave prefix
// sum.  The caller syncs the wave's LDS before reading the list.
template <typename Load4>
__device__ __forceinline__ int compact_segment(int s0, int t, float thr, Load4& load4, int* list) {
  const int lane = lane_id();
  const int sb = s0 + 8 * lane;
  float sv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (sb <= t) {
    float a4[4];
    load4(sb, a4);
#pragma unroll
    for (int c = 0; c < 4; ++c) sv[c] = a4[c];
    if (sb + 4 <= t) {
      load4(sb + 4, a4);
#pragma unroll
      for (int c = 0; c < 4; ++c) sv[4 + c] = a4[c];
    }
  }
  int cnt = 0;
  bool keep[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    keep[c] = (sb + c <= t) && (sv[c] >= thr);
    cnt += keep[c] ? 1 : 0;
  }
  const int incl = wave_inclusive_sum(cnt);
  const int total = wave_read_lane(incl, kWave - 1);
  int p = incl - cnt;
#pragma unroll
  for (int c = 0; c < 8; ++c)
    if (keep[c]) list[p++] = sb + c;
  return total;
}

// This lane's slice of query row t, times scale_log2 (0 past the row).
// EQ: elements the wave covers (its heads times DQ); RQ: elements from one
// query row to the next (EQ, or HQ*DQ when the wave covers a head chunk).
template <typename Tag, int EK>
__device__ __forceinline__ void load_query(const typename Tag::raw* __restrict__ Q, int t,
                                           int EQ, float scale_log2, float (&q)[EK],
                                           int RQ = 0) {
  const int lane = lane_id();
  if (lane * EK < EQ) {
    load_cvt<Tag, EK>(Q + static_cast<int64_t>(t) * (RQ > 0 ? RQ : EQ) + lane * EK, q);
#pragma unroll
    for (int e = 0; e < EK; ++e) q[e] *= scale_log2;
  } else {
#pragma unroll
    for (int e = 0; e < EK; ++e) q[e] = 0.f;
  }
}

// Q/K/V point at this batch element: Q row t is Q + t*HQ*DQ, etc.
// load4(s, sv) loads scores s..s+3 (s <= t, s % 4 == 0) of this query's row.
// qpre: this lane's query slice from load_query, loaded early by the caller
// (nullptr: loaded here).  PIPE: overlap each group's loads with the
// neighbouring group's arithmetic (below); it needs more registers, which
// the fused kernel has to spare and the gather kernel's occupancy does not.
// Head chunks: HQ may be a subset of a row's heads (rows too wide for one
// wave's registers).  Then Q/K/V/out_row point at the chunk's first head
// and RQ / RV give the full row lengths (elements of a Q or K row, of a V
// row); 0 means the row is exactly the HQ heads.
template <typename Tag, int EK, int EV, bool PIPE = false, typename Load4>
__device__ __forceinline__ void attend_query(const typename Tag::raw* __restrict__ Q,
                                             const typename Tag::raw* __restrict__ K,
                                             const typename Tag::raw* __restrict__ V, int t,
                                             int HQ, int DQ, int DV, float scale_log2,
                                             float thr, Load4&& load4, int* list,
                                             float* __restrict__ out_row,
                                             const float* qpre = nullptr, int RQ = 0,
                                             int RV = 0) {
  using raw = typename Tag::raw;
  const int lane = lane_id();
  const int EQ = HQ * DQ;
  const int EVt = HQ * DV;
  const int rowq = RQ > 0 ? RQ : EQ;   // elements per Q / K row
  const int rowv = RV > 0 ? RV : EVt;  // elements per V row
  const bool kact = lane * EK < EQ;
  const bool vact = lane * EV < EVt;
  const int lphk = DQ / EK;                     // lanes per head, K side
  const int hv = (lane * EV) / DV;              // head of this lane's V slice
  const int src_lane = (hv * lphk) & (kWave - 1);
  const bool same_map = (DQ / EK) == (DV / EV);  // K and V slices cover the same head

  float q[EK];
  if (qpre != nullptr) {
#pragma unroll
    for (int e = 0; e < EK; ++e) q[e] = qpre[e];
  } else {
    load_query<Tag, EK>(Q, t, EQ, scale_log2, q, rowq);
  }
  float acc[EV];
#pragma unroll
  for (int e = 0; e < EV; ++e) acc[e] = 0.f;
  float m = -__builtin_huge_valf();
  float lsum = 0.f;

  // Keys gathered per group: as many as fit ~64 registers of K+V.
  constexpr int U = (EK + EV <= 4) ? 16 : (EK + EV <= 8) ? 8 : (EK + EV <= 16) ? 4 : 2;
  // Loads the K (or V) slices of keys ss[0..U) (entries past nu repeat key
  // ss[0] and are ignored by the caller): the group's list entries come in
  // with vector LDS reads, and every load takes a 32-bit byte offset against
  // the uniform K or V base (the host keeps a batch element's K and V under
  // 4 GiB) -- one offset register per key, so all of a group's loads fit in
  // flight together.  No load is predicated: lanes past the row
  // (EQ < 64*EK) read the row's start and contribute zero through q = 0 / an
  // unstored accumulator.
  constexpr uint32_t kRaw = sizeof(raw);
  const uint32_t koff_l = kact ? static_cast<uint32_t>(lane * EK) * kRaw : 0u;
  const uint32_t voff_l = vact ? static_cast<uint32_t>(lane * EV) * kRaw : 0u;
  const char* Kb = reinterpret_cast<const char*>(K);
  const char* Vb = reinterpret_cast<const char*>(V);
  auto group_keys = [&](const int* ss, int nu, uint32_t (&sidx)[U]) {
    int raw_idx[U];
    if constexpr (U % 4 == 0) {
#pragma unroll
      for (int i = 0; i < U / 4; ++i) {
        const int4 v4 = reinterpret_cast<const int4*>(ss)[i];
        raw_idx[4 * i] = v4.x; raw_idx[4 * i + 1] = v4.y; raw_idx[4 * i + 2] = v4.z; raw_idx[4 * i + 3] = v4.w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) raw_idx[u] = ss[u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) sidx[u] = static_cast<uint32_t>(u < nu ? raw_idx[u] : raw_idx[0]);
  };
  auto load_k = [&](const int* ss, int nu, float (&kv)[U][EK]) {
    uint32_t sidx[U];
    group_keys(ss, nu, sidx);
#pragma unroll
    for (int u = 0; u < U; ++u)
      load_cvt<Tag, EK>(reinterpret_cast<const raw*>(
                            Kb + (sidx[u] * (static_cast<uint32_t>(rowq) * kRaw) + koff_l)),
                        kv[u]);
  };
  auto load_v = [&](const int* ss, int nu, float (&vv)[U][EV]) {
    uint32_t sidx[U];
    group_keys(ss, nu, sidx);
#pragma unroll
    for (int u = 0; u < U; ++u)
      load_cvt<Tag, EV>(reinterpret_cast<const raw*>(
                            Vb + (sidx[u] * (static_cast<uint32_t>(rowv) * kRaw) + voff_l)),
                        vv[u]);
  };
  auto load_kv = [&](const int* ss, int nu, float (&kv)[U][EK], float (&vv)[U][EV]) {
    uint32_t sidx[U];
    group_keys(ss, nu, sidx);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t rk = sidx[u] * (static_cast<uint32_t>(rowq) * kRaw);
      const uint32_t rv = (rowq == rowv) ? rk : sidx[u] * (static_cast<uint32_t>(rowv) * kRaw);
      load_cvt<Tag, EK>(reinterpret_cast<const raw*>(Kb + (rk + koff_l)), kv[u]);
      load_cvt<Tag, EV>(reinterpret_cast<const raw*>(Vb + (rv + voff_l)), vv[u]);
    }
  };
  // Each group is two halves: logits and the softmax update from K (A), then
  // the P*V accumulation from V (B).  With PIPE the loop below issues a
  // group's V loads before its half A and the next group's K loads before
  // its half B, so each load overlaps the other half's arithmetic and the
  // other load's wait (the K slices are dead after half A).

  // General form: per-key logits summed over the head's lanes.
  float lg[U];
  float mnew_g = 0.f;
  auto half_a = [&](int nu, const float (&kv)[U][EK]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EK; ++e) d = fmaf(q[e], kv[u][e], d);
      lg[u] = d;
    }
    // sum over the head's lphk lanes: DPP inside 16-lane rows, LDS
    // permutes across rows
    auto head_sum = [&](auto step) {
      constexpr int W = decltype(step)::value;
      if (lphk > W) {
#pragma unroll
        for (int u = 0; u < U; ++u) lg[u] += dpp_partner<W>(lg[u]);
      }
    };
    head_sum(std::integral_constant<int, 1>{});
    head_sum(std::integral_constant<int, 2>{});
    head_sum(std::integral_constant<int, 4>{});
    head_sum(std::integral_constant<int, 8>{});
    for (int o = 16; o < lphk; o <<= 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) lg[u] += __shfl_xor(lg[u], o, kWave);
    }
    if (!same_map) {
#pragma unroll
      for (int u = 0; u < U; ++u) lg[u] = __shfl(lg[u], src_lane, kWave);
    }
    float mnew = m;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (u < nu) mnew = fmaxf(mnew, lg[u]);
    const float alpha = exp2f(m - mnew);
    lsum *= alpha;
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[e] *= alpha;
    m = mnew;
    mnew_g = mnew;
  };
  auto half_b = [&](int nu, const float (&vv)[U][EV]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u < nu) {
        // bare v_exp_f32: results below 2^-126 flush to 0, which no sum can see
        const float p = __builtin_amdgcn_exp2f(lg[u] - mnew_g);
        lsum += p;
#pragma unroll
        for (int e = 0; e < EV; ++e) acc[e] = fmaf(p, vv[u][e], acc[e]);
      }
    }
  };

  // Variant for heads spanning exactly U lanes (K and V slices on the same
  // lanes): a reduce-scatter sums the U partial dot products so that lane j
  // of a head ends up holding the logit of key j (U-1 shuffles instead of
  // U*log2(U)); the softmax then takes one exp per lane, and the U
  // probabilities are broadcast back for the P*V accumulation.  The
  // per-lane normaliser holds only the lane's own keys until the end.
  float lpart = 0.f;
  float p_own = 0.f;
  auto half_a_rs = [&](int nu, const float (&kv)[U][EK]) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EK; ++e) d = fmaf(q[e], kv[u][e], d);
      v[u] = d;
    }
    // after the step of width w, lane j keeps the half of its keys selected
    // by bit w of j: lane j ends with key j of the group.  The partner lane
    // (DPP, inside the row) has the other bit w and the same higher bits.
    auto rs_step = [&](auto step) {
      constexpr int W = decltype(step)::value;
      if constexpr (W < U) {
        constexpr int cur = 2 * W;
        const bool up = (lane & W) != 0;
#pragma unroll
        for (int i = 0; i < cur / 2; ++i) {
          const float keep = up ? v[cur / 2 + i] : v[i];
          const float send = up ? v[i] : v[cur / 2 + i];
          v[i] = keep + dpp_partner<W>(send);
        }
      }
    };
    rs_step(std::integral_constant<int, 8>{});
    rs_step(std::integral_constant<int, 4>{});
    rs_step(std::integral_constant<int, 2>{});
    rs_step(std::integral_constant<int, 1>{});
    const int j = lane & (U - 1);
    const float lgj = (j < nu) ? v[0] : -__builtin_huge_valf();
    float mx = lgj;
    if constexpr (U > 1) mx = fmaxf(mx, dpp_partner<1>(mx));
    if constexpr (U > 2) mx = fmaxf(mx, dpp_partner<2>(mx));
    if constexpr (U > 4) mx = fmaxf(mx, dpp_partner<4>(mx));
    if constexpr (U > 8) mx = fmaxf(mx, dpp_partner<8>(mx));
    const float mnew = fmaxf(m, mx);
    const float alpha = exp2f(m - mnew);
    p_own = (j < nu) ? __builtin_amdgcn_exp2f(lgj - mnew) : 0.f;
    lpart = fmaf(lpart, alpha, p_own);
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[e] *= alpha;
    m = mnew;
  };
  auto half_b_rs = [&](int nu, const float (&vv)[U][EV]) {
    auto bcast_acc = [&](auto uc) {
      constexpr int UU = decltype(uc)::value;
      if constexpr (UU < U) {
        if (UU < nu) {
          const float p = group_bcast<U, UU>(p_own);
#pragma unroll
          for (int e = 0; e < EV; ++e) acc[e] = fmaf(p, vv[UU][e], acc[e]);
        }
      }
    };
    [&]<int... Us>(std::integer_sequence<int, Us...>) {
      (bcast_acc(std::integral_constant<int, Us>{}), ...);
    }(std::make_integer_sequence<int, 16>{});
  };
  // reduce-scatter needs every lane active on both sides (EQ = EVt = 64*E)
  const bool use_rs = same_map && lphk == U && EK == EV && EQ == kWave * EK && EVt == kWave * EV;

  // All groups of one list segment.  PIPE: K of the first group, then per
  // group V loads, half A, the next group's K loads, half B.  Otherwise a
  // group's K and V loads, then both halves: one memory round trip each.
  float kv[U][EK];
  float vv[U][EV];
  auto run_groups = [&](int total, auto&& ha, auto&& hb) {
    if (total <= 0) return;
    if constexpr (PIPE) {
      load_k(list, min(U, total), kv);
      for (int i = 0; i < total; i += U) {
        const int nu = min(U, total - i);
        load_v(list + i, nu, vv);
        ha(nu, kv);
        if (i + U < total) load_k(list + i + U, min(U, total - i - U), kv);
        hb(nu, vv);
      }
    } else {
      for (int i = 0; i < total; i += U) {
        const int nu = min(U, total - i);
        load_kv(list + i, nu, kv, vv);
        ha(nu, kv);
        hb(nu, vv);
      }
    }
  };

  for (int s0 = 0; s0 <= t; s0 += kListCap) {
    const int total = compact_segment(s0, t, thr, load4, list);
    wave_lds_sync();
    if (use_rs) run_groups(total, half_a_rs, half_b_rs);
    else run_groups(total, half_a, half_b);
    wave_lds_sync();
  }
  if (use_rs) {
    float ls = lpart;
    if constexpr (U > 1) ls += dpp_partner<1>(ls);
    if constexpr (U > 2) ls += dpp_partner<2>(ls);
    if constexpr (U > 4) ls += dpp_partner<4>(ls);
    if constexpr (U > 8) ls += dpp_partner<8>(ls);
    lsum = ls;
  }

  if (vact) {
    const float inv = 1.f / lsum;  // lsum == 0 only if nothing passed: NaN, as the reference
#pragma unroll
    for (int e = 0; e < EV; ++e) out_row[lane * EV + e] = acc[e] * inv;
  }
}

// Elements [4j, 4j + 4), j = lane % 32, of fp32 query row t (rows of 128
// elements), times scale_log2: attend_query_pair's slice.
__device__ __forceinline__ void load_query_pair(const float* __restrict__ Q, int t, float scale_log2,
                                                float (&q)[4]) {
  const float4 f =
      *reinterpret_cast<const float4*>(Q + static_cast<int64_t>(t) * 128 + 4 * (lane_id() & 31));
  q[0] = f.x * scale_log2;
  q[1] = f.y * scale_log2;
  q[2] = f.z * scale_log2;
  q[3] = f.w * scale_log2;
}

// attend_query for fp32 rows of exactly 128 elements (HQ*DQ = HQ*DV = 128,
// DQ = DV, DQ % 4 == 0; Q, K, V and out 16-byte aligned), two keys per gather
// instruction.  Lane l owns elements [4j, 4j + 4), j = l % 32, of a row; in
// load i of a group the lower half-wave reads key 2i of the group and the
// upper half key 2i + 1, so one wave load moves 16 bytes per lane (two
// 512-byte rows) where attend_query moves 8 (one row).  A CU issues random-row
// gathers at about one wave load per 15 cycles whatever their width up to 16
// bytes per lane (a probe of L2-resident random rows on gfx950: ~35 bytes per
// cycle per CU with 8-byte lanes, ~62 with 16-byte lanes), so two rows per
// load halve the gather instructions.  A head spans DQ/4 lanes of a half and
// its logit is a butterfly over them.  The running max is shared by the two
// halves (one lane exchange per group of 16 keys); each half sums the
// probabilities and P*V of the keys it read, and the halves' sums are added
// at the end.  Same selection and result as attend_query (the sums are
// ordered differently: rounding differs at the last bits).  A group's K and
// V loads go out together (overlapping them with the neighbouring group's
// arithmetic, as attend_query's PIPE form does, measured 2% slower here: the
// gathers are bound by the CU's load issue, not by their latency).
template <typename Load4>
__device__ __forceinline__ void attend_query_pair(const float* __restrict__ Q,
                                                  const float* __restrict__ K,
                                                  const float* __restrict__ V, int t, int DQ,
                                                  float scale_log2, float thr, Load4&& load4,
                                                  int* list, float* __restrict__ out_row,
                                                  const float* qpre = nullptr) {
  constexpr uint32_t kRowBytes = 128 * 4;
  constexpr int NL = 8;  // loads per group: 16 keys
  const int lane = lane_id();
  const int half = lane >> 5;
  const int j4 = 4 * (lane & 31);
  const int lph = DQ / 4;  // lanes per head
  float q[4];
  if (qpre != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = qpre[e];
  } else {
    load_query_pair(Q, t, scale_log2, q);
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_huge_valf();
  float lsum = 0.f;
  const uint32_t off_l = static_cast<uint32_t>(j4) * 4u;
  const char* Kb = reinterpret_cast<const char*>(K);
  const char* Vb = reinterpret_cast<const char*>(V);
  // Load i reads key 2i + half of the group's list entries ss[0..nu); entries
  // past nu read key ss[0] and are masked (ok = false).  The list comes in
  // with vector LDS reads (every lane the same 16 entries); every load takes
  // a 32-bit byte offset against the uniform base (the host keeps a batch
  // element's K and V under 4 GiB).
  auto load_rows = [&](const char* base, const int* ss, int nu, float (&r)[NL][4],
                       bool (&ok)[NL]) {
    int raw_idx[2 * NL];
#pragma unroll
    for (int i = 0; i < NL / 2; ++i) {
      const int4 v4 = reinterpret_cast<const int4*>(ss)[i];
      raw_idx[4 * i] = v4.x; raw_idx[4 * i + 1] = v4.y; raw_idx[4 * i + 2] = v4.z; raw_idx[4 * i + 3] = v4.w;
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      ok[i] = 2 * i + half < nu;
      const int s = half ? raw_idx[2 * i + 1] : raw_idx[2 * i];
      const uint32_t sidx = static_cast<uint32_t>(ok[i] ? s : raw_idx[0]);
      const float4 f = *reinterpret_cast<const float4*>(base + (sidx * kRowBytes + off_l));
      r[i][0] = f.x; r[i][1] = f.y; r[i][2] = f.z; r[i][3] = f.w;
    }
  };
  float lg[NL];
  // Logits of the group's keys and the softmax rescale (from K).
  auto half_a = [&](const bool (&ok)[NL], const float (&kv)[NL][4]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) d = fmaf(q[e], kv[i][e], d);
      lg[i] = d;
    }
    auto head_sum = [&](auto step) {
      constexpr int W = decltype(step)::value;
      if (lph > W) {
#pragma unroll
        for (int i = 0; i < NL; ++i) lg[i] += dpp_partner<W>(lg[i]);
      }
    };
    head_sum(std::integral_constant<int, 1>{});
    head_sum(std::integral_constant<int, 2>{});
    head_sum(std::integral_constant<int, 4>{});
    head_sum(std::integral_constant<int, 8>{});
    if (lph > 16) {
#pragma unroll
      for (int i = 0; i < NL; ++i) lg[i] = sum_xor16(lg[i]);
    }
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      lg[i] = ok[i] ? lg[i] : -__builtin_huge_valf();
      mx = fmaxf(mx, lg[i]);
    }
    const float mnew = fmaxf(m, max_xor32(mx));  // over both halves' keys
    const float alpha = exp2f(m - mnew);
    lsum *= alpha;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= alpha;
    m = mnew;
  };
  // P*V of the group's keys (from V).
  auto half_b = [&](const bool (&ok)[NL], const float (&vv)[NL][4]) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      // bare v_exp_f32: results below 2^-126 flush to 0, which no sum can see
      const float p = ok[i] ? __builtin_amdgcn_exp2f(lg[i] - m) : 0.f;
      lsum += p;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(p, vv[i][e], acc[e]);
    }
  };
  float kv[NL][4], vv[NL][4];
  bool okk[NL], okv[NL];
  for (int s0 = 0; s0 <= t; s0 += kListCap) {
    const int total = compact_segment(s0, t, thr, load4, list);
    wave_lds_sync();
    for (int i = 0; i < total; i += 2 * NL) {
      const int nu = min(2 * NL, total - i);
      load_rows(Kb, list + i, nu, kv, okk);
      load_rows(Vb, list + i, nu, vv, okv);
      half_a(okk, kv);
      half_b(okv, vv);
    }
    wave_lds_sync();
  }
  lsum = sum_xor32(lsum);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = sum_xor32(acc[e]);
  if (half == 0) {
    const float inv = 1.f / lsum;  // lsum == 0 only if nothing passed: NaN, as the reference
    *reinterpret_cast<float4*>(out_row + j4) =
        make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
  }
}

}  // namespace dsa
