// staged_attn.hip -- threshold-driven sparse attention with K/V rows staged
// through LDS, for long rows (gfx950).
//
// Same result as sparse_attn.hip (reference dsa_attention.py:234-324):
//   sel(t,s) = s <= t && scores[t,s] >= thr[t]
//   O[t,h,:] = sum_{s in sel} softmax_s(<Q[t,h],K[s,h]> * scale) V[s,h,:]
// but organised around the keys instead of the queries.  When every query of
// a long row selects a few hundred keys (config 3: k = 256 of up to 4096),
// the per-query gather pulls each query's K/V rows from L2/MALL on its own
// (16.6 GB per forward at config 3) although the selected sets of nearby
// queries are spread over the same key range.  Here a block streams its
// causal key range once, in tiles of 16 KiB of K rows (8 or 16 keys) copied
// HBM/L2 -> LDS by the DMA path (global_load_lds, a ring of 4 slots, 3 tiles
// ahead), and every wave computes its queries' selected pairs of the tile
// from LDS.
//
// Block = 16 waves = two 32-query tiles of one batch element, tile p and
// tile ntile-1-p, so every block has about the same causal work (T keys x 32
// queries) and the short tile's keys come with the long tile's stream.  Wave
// w owns queries 2w, 2w+1 of each tile.  Per key tile a wave reads its 4
// queries' scores (one per lane, copied with the tile), turns them into a
// 64-bit selection mask, and walks the keys any of its queries selected: it
// reads the key's K and V slices from LDS once and updates each selecting
// query.
//
// Measured at config 3 (B=4, T=4096, k=256, HQ=8, D=64, fp32): 0.54 ms
// against 0.69-0.75 ms for per-query gathers; at T=2047 the gathers are
// faster (0.31 vs 0.38 ms), so the threshold entry point switches at 3072.
// What limits it: the barrier per key tile waits for the busiest wave (the
// selected pairs per wave and tile vary about 1.7x around their mean).
//
// Lane layout as in attn_tile.h: a K (or V) row is 64*E elements, lane l
// owns [l*E, (l+1)*E); a head spans DQ/E lanes and its logit is a butterfly
// over them.  Softmax is online in the log2 domain with fp32 state; the
// running max moves only when a logit exceeds it by more than 2^8, so the
// accumulator is rescaled on a few keys per query.  Rows that select
// nothing output NaN (0/0), as the reference.
#include <type_traits>

#include "dsa_device.h"
#include "dsa_launch.h"

namespace dsa {
namespace {

constexpr int kSTQ = 32;     // queries per tile; a block holds two tiles
constexpr int kSlots = 4;    // LDS ring of key tiles: DMA runs 3 tiles ahead
constexpr int kSlotK = 16384;  // bytes of K (and of V) per key tile

#define DSA_LDS __attribute__((address_space(3)))

struct StagedArgs {
  const float* scores;
  int64_t ld;
  const float* thr;
  const void* Q;
  const void* K;
  const void* V;
  int64_t B;
  int T;
  int DQ;          // head dim (DQ = DV); a row holds 64*E / DQ heads
  float scale_log2;
  float* out;
  int ntile;       // ceil(T / kSTQ)
};

template <typename Tag, int E>
constexpr int row_bytes() { return kWave * E * Tag::kBytes; }
// Keys per LDS tile: 16 KiB of K rows (8 keys of 512 fp32, 16 otherwise).
template <typename Tag, int E>
constexpr int tile_keys() { return kSlotK / row_bytes<Tag, E>(); }

// LDS row layout.  A lane reads its slice of a row as E*bytes/16 chunks of
// 16 bytes.  With one chunk per lane the row is stored as is (lane l reads
// chunk l: 64 consecutive chunks, no bank conflict).  With two (fp32, E = 8)
// the even chunks go to the first half of the row and the odd ones to the
// second, so the wave's two reads are each 64 consecutive chunks too
// (stored as is, lanes l and l+8 would hit the same banks: 48.6% of LDS
// cycles were conflicts).
template <typename Tag, int E>
constexpr int chunks_per_lane() { return E * Tag::kBytes / 16; }

// Logical chunk (16 bytes of the row in memory order) held at physical
// position pc of an LDS row of cpr chunks.
template <int CPL>
__device__ __forceinline__ int logical_chunk(int pc, int cpr) {
  if constexpr (CPL == 2) return pc < cpr / 2 ? 2 * pc : 2 * (pc - cpr / 2) + 1;
  else return pc;
}

// Copies rows s0 .. s0+KT-1 of one batch element's [T, 64E] K or V into
// dst (rows past T repeat row T-1; they are never selected) with the NT
// threads of the block, in the LDS row layout above.  Physical chunk c of
// the tile (16 bytes) lands at dst + 16c: each wave instruction fills 1 KiB.
template <typename Tag, int E, int NT, int KT>
__device__ __forceinline__ void dma_rows(const char* __restrict__ src, int s0, int T,
                                         DSA_LDS uint8_t* dst, int tid) {
  constexpr int RB = row_bytes<Tag, E>();
  constexpr int NCH = KT * RB / 16;
  constexpr int CPR = RB / 16;  // chunks per row
#pragma unroll
  for (int c0 = 0; c0 < NCH; c0 += NT) {
    if (c0 + (tid & ~(kWave - 1)) < NCH) {  // whole waves only
      const int c = c0 + tid;
      const int r = c / CPR;
      const uint32_t s = static_cast<uint32_t>(min(s0 + r, T - 1));
      const int lc = logical_chunk<chunks_per_lane<Tag, E>()>(c % CPR, CPR);
      const uint32_t off = s * static_cast<uint32_t>(RB) + 16u * static_cast<uint32_t>(lc);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(src + off),
                                       dst + (c0 + (tid & ~(kWave - 1))) * 16, 16, 0, 0);
    }
  }
}

// This lane's E elements of an LDS row (layout above), as fp32.
template <typename Tag, int E>
__device__ __forceinline__ void lds_slice(const DSA_LDS uint8_t* row, int lane, float (&v)[E]) {
  if constexpr (Tag::kBytes == 4) {
    static_assert(E == 4 || E == 8, "one or two chunks per lane");
    const DSA_LDS f32x4* p = reinterpret_cast<const DSA_LDS f32x4*>(row);
    const f32x4 f = p[lane];
    v[0] = f[0]; v[1] = f[1]; v[2] = f[2]; v[3] = f[3];
    if constexpr (E == 8) {
      const f32x4 h = p[kWave + lane];  // odd chunks: second half of the row
      v[4] = h[0]; v[5] = h[1]; v[6] = h[2]; v[7] = h[3];
    }
  } else {
    static_assert(E == 8, "one chunk per lane");
    const DSA_LDS uint16_t* p = reinterpret_cast<const DSA_LDS uint16_t*>(row) + lane * E;
#pragma unroll
    for (int i = 0; i < E; i += 8) {
      const u32x4 u = *reinterpret_cast<const DSA_LDS u32x4*>(p + i);
      const uint32_t w[4] = {u[0], u[1], u[2], u[3]};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[i + 2 * j] = to_f32(Tag{}, static_cast<uint16_t>(w[j] & 0xffffu));
        v[i + 2 * j + 1] = to_f32(Tag{}, static_cast<uint16_t>(w[j] >> 16));
      }
    }
  }
}

// LPH: lanes per head (DQ / E), a compile-time constant so that the head
// butterfly is straight-line code.  QPW: queries per wave (QPW/2 from each
// tile); the block has 64/QPW waves.
//
// Pipeline: kSlots LDS slots, each holding one key tile's K rows, V rows and
// the block's scores for it, all copied by DMA.  Iteration kt waits for
// tile kt's copies, passes one barrier (every wave is then done with tile
// kt-1, whose slot is free), issues the copies of tile kt+3 into that slot
// and computes tile kt.  Every iteration issues the same copies (tiles past
// the end copy clamped rows into a slot nobody reads), so the wait is one
// fixed vmcnt: all but the 2 tiles' copies issued after tile kt's.  The
// slots are separate LDS objects and the loop is unrolled over them, so the
// compiler sees that a copy into one slot does not alias reads of another
// and leaves the copies in flight.
template <typename Tag, int E, int LPH, int QPW>
__global__ __launch_bounds__(64 / QPW * kWave) void staged_attn_kernel(StagedArgs a) {
  static_assert(QPW == 4 || QPW == 8, "4 or 8 queries per wave");
  constexpr int NW = 64 / QPW;           // waves per block
  constexpr int NT = NW * kWave;         // threads per block
  constexpr int HALF = QPW / 2;          // queries per wave from each tile
  constexpr int KT = tile_keys<Tag, E>();
  static_assert(KT == 8 || KT == 16, "8 or 16 keys per tile");
  static_assert(QPW * KT <= kWave, "one score per lane per tile");
  constexpr int DKV = 2 * ((kSlotK / 16 + NT - 1) / NT);  // K and V copy instructions per tile
  constexpr int WAITN = 2 * (DKV + 1);                    // + 1 score copy per tile
  static_assert(WAITN <= 63, "vmcnt field");
  using raw = typename Tag::raw;
  constexpr int RB = row_bytes<Tag, E>();
  constexpr int RE = kWave * E;  // elements per K/V row
  constexpr int SCB = NW * kWave * 4;  // score bytes per tile (one float per lane)
  // One LDS object per slot (K rows, V rows, scores): four objects keep the
  // compiler's tracking of copies in flight exact.
  struct Slot {
    uint8_t k[kSlotK];
    uint8_t v[kSlotK];
    uint8_t c[SCB];
  };
  __shared__ __align__(16) Slot sl0, sl1, sl2, sl3;
  DSA_LDS uint8_t* ks[kSlots] = {(DSA_LDS uint8_t*)sl0.k, (DSA_LDS uint8_t*)sl1.k,
                                 (DSA_LDS uint8_t*)sl2.k, (DSA_LDS uint8_t*)sl3.k};
  DSA_LDS uint8_t* vs[kSlots] = {(DSA_LDS uint8_t*)sl0.v, (DSA_LDS uint8_t*)sl1.v,
                                 (DSA_LDS uint8_t*)sl2.v, (DSA_LDS uint8_t*)sl3.v};
  DSA_LDS uint8_t* cs[kSlots] = {(DSA_LDS uint8_t*)sl0.c, (DSA_LDS uint8_t*)sl1.c,
                                 (DSA_LDS uint8_t*)sl2.c, (DSA_LDS uint8_t*)sl3.c};

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = lane_id();
  const int T = a.T;
  const int64_t b = static_cast<int64_t>(blockIdx.x) % a.B;
  const int p = static_cast<int>(static_cast<int64_t>(blockIdx.x) / a.B);
  const int ta = p, tb = a.ntile - 1 - p;  // ta <= tb

  // Query i of this wave: HALF*wave + i % HALF of tile ta (i < HALF) or of
  // tile tb (unless the pair is one tile).
  auto query_of = [&](int i) { return (i < HALF ? ta : tb) * kSTQ + HALF * wave + (i % HALF); };
  auto valid = [&](int i, int t) { return t < T && (i < HALF || tb != ta); };
  const int s_end = min(T, (tb + 1) * kSTQ);  // keys any query of the block reaches
  const int nkt = (s_end + KT - 1) / KT;

  // This lane's score per key tile: query lane / KT of the wave (lanes past
  // the wave's QPW queries load a clamped entry and select nothing), key
  // s0 + lane % KT, clamped into the row (the mask tests causality).
  const int j_l = lane % KT;
  const int i_l = lane / KT;
  const int t_l = (i_l < HALF ? ta : tb) * kSTQ + HALF * wave + (i_l % HALF);
  const bool v_l = i_l < QPW && t_l < T && (i_l < HALF || tb != ta);
  const int tc_l = min(t_l, T - 1);
  const float thr_l = a.thr[b * T + tc_l];
  const char* srow = reinterpret_cast<const char*>(a.scores + (b * T + tc_l) * a.ld);
  const int64_t s_clamp = a.ld - 1;

  const char* Kb = static_cast<const char*>(a.K) + b * T * static_cast<int64_t>(RB);
  const char* Vb = static_cast<const char*>(a.V) + b * T * static_cast<int64_t>(RB);
  auto copy_tile = [&](auto slot_c, int t) {
    constexpr int S = decltype(slot_c)::value;
    dma_rows<Tag, E, NT, KT>(Kb, t * KT, T, ks[S], tid);
    dma_rows<Tag, E, NT, KT>(Vb, t * KT, T, vs[S], tid);
    const int64_t s = min<int64_t>(static_cast<int64_t>(t) * KT + j_l, s_clamp);
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(srow + 4 * s),
                                     cs[S] + wave * (kWave * 4), 4, 0, 0);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  copy_tile(S0{}, 0);
  copy_tile(S1{}, 1);
  copy_tile(S2{}, 2);

  // Query slices (times scale_log2).
  const raw* Qb = static_cast<const raw*>(a.Q) + b * T * static_cast<int64_t>(RE);
  float q[QPW][E];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int tl = min(query_of(i), T - 1);
    load_cvt<Tag, E>(Qb + static_cast<int64_t>(tl) * RE + lane * E, q[i]);
#pragma unroll
    for (int e = 0; e < E; ++e) q[i][e] *= a.scale_log2;
  }

  float acc[QPW][E];
  float m[QPW], l[QPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    m[i] = -__builtin_huge_valf();
    l[i] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[i][e] = 0.f;
  }

  auto head_sum = [&](float x) {
    if constexpr (LPH > 1) x += dpp_partner<1>(x);
    if constexpr (LPH > 2) x += dpp_partner<2>(x);
    if constexpr (LPH > 4) x += dpp_partner<4>(x);
    if constexpr (LPH > 8) x += dpp_partner<8>(x);
    if constexpr (LPH > 16) x = sum_xor16(x);  // both lanes get own + partner
    if constexpr (LPH > 32) x = sum_xor32(x);
    return x;
  };

  // One key tile in slot S: the selection from its scores, then the keys any
  // of the wave's queries selected.  With 4 elements per lane, two at a time
  // (the next key's K/V slices are read from LDS while the current one is
  // used; the reads are unconditional -- row 0 when there is no next key --
  // so the wait for the current key's slices can leave the next key's reads
  // in flight).
  auto tile = [&](auto slot_c, int kt) {
    constexpr int S = decltype(slot_c)::value;
    // Tile kt landed everywhere, and every wave is done with tile kt-1: this
    // wave's copies of tile kt are complete, then the barrier.  (A release
    // fence here would also wait for the copies still in flight.  Every LDS
    // read of tile kt-1 fed values this wave has already used.)
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    const int s0 = kt * KT;
    const float sc = *reinterpret_cast<const DSA_LDS float*>(cs[S] + wave * (kWave * 4) + lane * 4);
    // bit i*KT + j: query i of the wave selects key s0 + j (NaN scores and
    // thresholds select nothing)
    const uint64_t sel = ballot(v_l && s0 + j_l <= t_l && sc >= thr_l);
    copy_tile(std::integral_constant<int, (S + 3) % kSlots>{}, kt + 3);
    uint32_t u;
    if constexpr (KT == 16) u = static_cast<uint32_t>((sel | (sel >> 16) | (sel >> 32) | (sel >> 48)) & 0xffffu);
    else u = static_cast<uint32_t>((sel | (sel >> 8) | (sel >> 16) | (sel >> 24)) & 0xffu);
    const DSA_LDS uint8_t* kl = ks[S];
    const DSA_LDS uint8_t* vl = vs[S];
    auto process = [&](int j, const float (&kv)[E], const float (&vv)[E]) {
#pragma unroll
      for (int i = 0; i < QPW; ++i) {
        if ((sel >> (i * KT + j)) & 1u) {
          float x = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) x = fmaf(q[i][e], kv[e], x);
          x = head_sum(x);
          const bool up = x > m[i] + 8.f;
          if (ballot(up) != 0u) {
            const float mn = up ? x : m[i];
            const float alpha = exp2f(m[i] - mn);  // m = -inf: 0 on an empty state
            l[i] *= alpha;
#pragma unroll
            for (int e = 0; e < E; ++e) acc[i][e] *= alpha;
            m[i] = mn;
          }
          // bare v_exp_f32: results below 2^-126 flush to 0, which no sum can see
          const float pr = __builtin_amdgcn_exp2f(x - m[i]);
          l[i] += pr;
#pragma unroll
          for (int e = 0; e < E; ++e) acc[i][e] = fmaf(pr, vv[e], acc[i][e]);
        }
      }
    };
    auto pop = [&]() {
      const int j = u != 0u ? __builtin_ctz(u) : -1;
      u &= u - 1u;
      return j;
    };
    if constexpr (E <= 4) {
      float ka[E], va[E], kb2[E], vb2[E];
      int j0 = pop();
      if (j0 >= 0) {
        lds_slice<Tag, E>(kl + j0 * RB, lane, ka);
        lds_slice<Tag, E>(vl + j0 * RB, lane, va);
      }
      while (j0 >= 0) {
        const int j1 = pop();
        lds_slice<Tag, E>(kl + max(j1, 0) * RB, lane, kb2);
        lds_slice<Tag, E>(vl + max(j1, 0) * RB, lane, vb2);
        process(j0, ka, va);
        if (j1 < 0) break;
        j0 = pop();
        lds_slice<Tag, E>(kl + max(j0, 0) * RB, lane, ka);
        lds_slice<Tag, E>(vl + max(j0, 0) * RB, lane, va);
        process(j1, kb2, vb2);
      }
    } else {
      // 8 elements per lane: no registers for a second key's slices
      for (int j = pop(); j >= 0; j = pop()) {
        float ka[E], va[E];
        lds_slice<Tag, E>(kl + j * RB, lane, ka);
        lds_slice<Tag, E>(vl + j * RB, lane, va);
        process(j, ka, va);
      }
    }
  };
  // Four tiles per trip: one per slot.
  for (int kt = 0; kt < nkt; kt += kSlots) {
    tile(S0{}, kt);
    if (kt + 1 >= nkt) break;
    tile(S1{}, kt + 1);
    if (kt + 2 >= nkt) break;
    tile(S2{}, kt + 2);
    if (kt + 3 >= nkt) break;
    tile(S3{}, kt + 3);
  }
  // the copies issued past the end must land before the block exits
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int t = query_of(i);
    if (valid(i, t)) {
      const float inv = 1.f / l[i];  // l == 0 only if nothing passed: NaN, as the reference
      float* orow = a.out + (b * T + t) * static_cast<int64_t>(RE) + lane * E;
#pragma unroll
      for (int e = 0; e < E; e += 4)
        *reinterpret_cast<float4*>(orow + e) =
            make_float4(acc[i][e] * inv, acc[i][e + 1] * inv, acc[i][e + 2] * inv,
                        acc[i][e + 3] * inv);
    }
  }
}

// Queries per wave by instance (4: 16 waves per block, 4 per SIMD; 8
// queries per wave and 2 waves per SIMD hid less latency).
template <typename Tag, int E>
constexpr int staged_qpw() { return 4; }

template <typename Tag, int E, int LPH>
hipError_t launch(const StagedArgs& a, hipStream_t stream) {
  constexpr int QPW = staged_qpw<Tag, E>();
  constexpr int NT = 64 / QPW * kWave;
  const int64_t npair = (a.ntile + 1) / 2;
  hipLaunchKernelGGL((staged_attn_kernel<Tag, E, LPH, QPW>), dim3(static_cast<unsigned>(a.B * npair)),
                     dim3(NT), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

bool staged_attn_supported(int dtype, int HQ, int DQ, int DV) {
  if (DQ != DV || HQ < 1 || DQ < 1) return false;
  const int64_t row = static_cast<int64_t>(HQ) * DQ;
  if (row % kWave != 0) return false;
  const int E = static_cast<int>(row / kWave);
  if (DQ % E != 0 || DQ / E > kWave) return false;  // a lane's slice stays inside one head
  if (dtype == 0) return E == 4 || E == 8;
  if (dtype == 1 || dtype == 2) return E == 8;
  return false;
}

hipError_t launch_staged_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, float scale, float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  StagedArgs a{scores, ld, thr, Q, K, V, B, static_cast<int>(T), DQ,
               scale * 1.4426950408889634f, out, static_cast<int>((T + kSTQ - 1) / kSTQ)};
  const int E = static_cast<int>(static_cast<int64_t>(HQ) * DQ / kWave);
  const int lph = DQ / E;
#define DSA_STAGED_LPH(Tag, e)                                      \
  switch (lph) {                                                    \
    case 1: return launch<Tag, e, 1>(a, stream);                    \
    case 2: return launch<Tag, e, 2>(a, stream);                    \
    case 4: return launch<Tag, e, 4>(a, stream);                    \
    case 8: return launch<Tag, e, 8>(a, stream);                    \
    case 16: return launch<Tag, e, 16>(a, stream);                  \
    case 32: return launch<Tag, e, 32>(a, stream);                  \
    case 64: return launch<Tag, e, 64>(a, stream);                  \
  }
  if (dtype == 0) {
    if (E == 4) { DSA_STAGED_LPH(F32, 4) }
    if (E == 8) { DSA_STAGED_LPH(F32, 8) }
  } else if (dtype == 1) {
    if (E == 8) { DSA_STAGED_LPH(BF16, 8) }
  } else if (dtype == 2) {
    if (E == 8) { DSA_STAGED_LPH(F16, 8) }
  }
#undef DSA_STAGED_LPH
  return hipErrorInvalidValue;
}

}  // namespace dsa
