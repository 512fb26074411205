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
// causal key range once, in tiles of 16 keys copied HBM/L2 -> LDS by the DMA
// path (buffer_load ... lds through range-checked buffer resources whose
// base moves with the tile, so a copy costs no per-lane address arithmetic;
// a ring of 4 slots, 3 tiles ahead, for rows of 1 KiB, and of 2 slots, 1
// tile ahead, for rows of 2 KiB), and every wave computes its queries'
// selected pairs of the tile from LDS.
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
// Measured at config 3 (B=4, T=4096, k=256, HQ=8, D=64, fp32): 0.438 ms
// against 0.69-0.75 ms for per-query gathers (8-key tiles in a ring of 4:
// 0.497 ms; with per-lane address arithmetic for the copies: 0.544 ms).
// What limits it: the barrier per key tile waits for the busiest wave (the
// selected pairs per wave and tile vary about 1.7x around their mean for
// 8-key tiles); 16-key tiles average the variation over twice the pairs.
// The threshold entry point takes this kernel only where it measured faster
// than the gathers (staged_attn_auto).
//
// Lane layout as in attn_tile.h: a K (or V) row is 64*E elements, lane l
// owns [l*E, (l+1)*E); a head spans DQ/E lanes and its logit is a butterfly
// over them.  Softmax is online in the log2 domain with fp32 state; the
// running max moves only when a logit exceeds it by more than 8 (a factor
// 2^8), so the accumulator is rescaled on a few keys per query.  Rows that select
// nothing output NaN (0/0), as the reference.
#include <type_traits>

#include "dsa_device.h"
#include "dsa_launch.h"

namespace dsa {
namespace {

constexpr int kSTQ = 32;     // queries per tile; a block holds two tiles

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
// Bytes of K (and of V) per key tile: 16 keys per tile.  A tile of 16 keys
// holds 16 KiB of K for rows of 1 KiB and 32 KiB for rows of 2 KiB (fp32,
// 512 elements); the LDS ring then has 4 or 2 slots.
template <typename Tag, int E>
constexpr int slot_bytes() { return 16 * row_bytes<Tag, E>(); }
template <typename Tag, int E>
constexpr int tile_keys() { return slot_bytes<Tag, E>() / row_bytes<Tag, E>(); }
template <typename Tag, int E>
constexpr int ring_slots() { return slot_bytes<Tag, E>() <= 16384 ? 4 : 2; }

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

// Byte offset, within a key tile of rows of RB bytes, of physical chunk c
// (16 bytes), which lands at LDS offset 16c in the row layout above: thread
// tid copies chunks tid, tid + NT, ..., so each wave instruction fills 1 KiB.
template <typename Tag, int E>
__device__ __forceinline__ uint32_t tile_chunk_offset(int c) {
  constexpr int RB = row_bytes<Tag, E>();
  constexpr int CPR = RB / 16;  // chunks per row
  const int lc = logical_chunk<chunks_per_lane<Tag, E>()>(c % CPR, CPR);
  return static_cast<uint32_t>((c / CPR) * RB + 16 * lc);
}

// Buffer resource over elements s0 .. n-1 of an array of `bytes`-sized
// elements (`base` is element 0; no element when s0 >= n): reads past
// element n-1 are range-checked by the hardware and return zeros.  The
// callers keep n * bytes below 2^31, so the size is 32-bit scalar
// arithmetic.  Word 3 is the raw-buffer configuration of CDNA.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const char* base, int s0, int n,
                                                           int bytes) {
  const int rem = s0 >= n ? 0 : (n - s0) * bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + static_cast<int64_t>(s0) * bytes,
                                           0, rem, 0x00020000);
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
// Pipeline: NS LDS slots (ring_slots), each holding one key tile's K rows,
// V rows and the block's scores for it, all copied by DMA.  Iteration kt
// waits for tile kt's copies, passes one barrier (every wave is then done
// with tile kt-1, whose slot is free), issues the copies of tile kt+NS-1
// into that slot and computes tile kt.  Every iteration issues the same
// copies (tiles past the end read as zeros into a slot nobody reads), so the
// wait is one fixed vmcnt: all but the copies of the NS-2 tiles issued after
// tile kt's.  The slots are separate LDS objects and the loop is unrolled
// over them, so the compiler sees that a copy into one slot does not alias
// reads of another and leaves the copies in flight.
template <typename Tag, int E, int LPH, int QPW>
__global__ __launch_bounds__(64 / QPW * kWave) void staged_attn_kernel(StagedArgs a) {
  static_assert(QPW == 4 || QPW == 8, "4 or 8 queries per wave");
  constexpr int NW = 64 / QPW;           // waves per block
  constexpr int NT = NW * kWave;         // threads per block
  constexpr int HALF = QPW / 2;          // queries per wave from each tile
  constexpr int KT = tile_keys<Tag, E>();
  static_assert(KT == 8 || KT == 16, "8 or 16 keys per tile");
  static_assert(QPW * KT <= kWave, "one score per lane per tile");
  constexpr int SK = slot_bytes<Tag, E>();
  constexpr int NS = ring_slots<Tag, E>();
  constexpr int CH = SK / 16 / NT;  // 16-byte chunks of K (and of V) per thread and tile
  static_assert(CH * 16 * NT == SK && (CH == 1 || CH == 2), "whole chunks per thread");
  constexpr int WAITN = (NS - 2) * (2 * CH + 1);  // copies of the tiles issued after tile kt
  static_assert(WAITN <= 63, "vmcnt field");
  using raw = typename Tag::raw;
  constexpr int RB = row_bytes<Tag, E>();
  constexpr int RE = kWave * E;  // elements per K/V row
  constexpr int SCB = NW * kWave * 4;  // score bytes per tile (one float per lane)
  // One LDS object per slot (K rows, V rows, scores): separate objects keep
  // the compiler's tracking of copies in flight exact.  With a ring of 2,
  // slots 2 and 3 are never referenced and take no LDS.
  struct Slot {
    uint8_t k[SK];
    uint8_t v[SK];
    uint8_t c[SCB];
  };
  __shared__ __align__(16) Slot sl0, sl1, sl2, sl3;
  DSA_LDS uint8_t* ks[4] = {(DSA_LDS uint8_t*)sl0.k, (DSA_LDS uint8_t*)sl1.k,
                            (DSA_LDS uint8_t*)sl2.k, (DSA_LDS uint8_t*)sl3.k};
  DSA_LDS uint8_t* vs[4] = {(DSA_LDS uint8_t*)sl0.v, (DSA_LDS uint8_t*)sl1.v,
                            (DSA_LDS uint8_t*)sl2.v, (DSA_LDS uint8_t*)sl3.v};
  DSA_LDS uint8_t* cs[4] = {(DSA_LDS uint8_t*)sl0.c, (DSA_LDS uint8_t*)sl1.c,
                            (DSA_LDS uint8_t*)sl2.c, (DSA_LDS uint8_t*)sl3.c};

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
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
  // key s0 + j_l is causal for this lane's query iff s0 <= lim_l (never for
  // lanes without a query)
  const int lim_l = v_l ? t_l - j_l : -1;

  // Copies go through buffer resources whose base moves with the tile (a
  // scalar computation): the per-lane offsets below are loop-invariant.  K
  // and V rows at or past T read as zeros (the resource ends at row T); they
  // are never causal.  A lane's score is element (tc_l, s0 + j_l) of this
  // batch element's [T, ld] rows; entries past the row's causal end read
  // whatever follows (the next row, or zeros past the last) and are masked
  // by lim_l.  The host keeps T*ld*4 below 2^31.
  uint32_t kv_off[CH];
#pragma unroll
  for (int r = 0; r < CH; ++r) kv_off[r] = tile_chunk_offset<Tag, E>(tid + r * NT);
  const uint32_t sc_off = static_cast<uint32_t>(tc_l) * static_cast<uint32_t>(a.ld) * 4u +
                          4u * static_cast<uint32_t>(j_l);
  const char* Kb = static_cast<const char*>(a.K) + b * T * static_cast<int64_t>(RB);
  const char* Vb = static_cast<const char*>(a.V) + b * T * static_cast<int64_t>(RB);
  const char* Sb = reinterpret_cast<const char*>(a.scores + b * T * a.ld);
  const int sc_elems = T * static_cast<int>(a.ld);  // < 2^29
  auto copy_tile = [&](auto slot_c, int t) __attribute__((always_inline)) {
    constexpr int S = decltype(slot_c)::value;
    const int s0 = t * KT;
    const __amdgpu_buffer_rsrc_t rk = span_rsrc(Kb, s0, T, RB);
    const __amdgpu_buffer_rsrc_t rv = span_rsrc(Vb, s0, T, RB);
#pragma unroll
    for (int r = 0; r < CH; ++r) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, ks[S] + r * NT * 16 + wave * 1024, 16,
                                               static_cast<int>(kv_off[r]), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, vs[S] + r * NT * 16 + wave * 1024, 16,
                                               static_cast<int>(kv_off[r]), 0, 0, 0);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(span_rsrc(Sb, s0, sc_elems, 4),
                                             cs[S] + wave * (kWave * 4), 4,
                                             static_cast<int>(sc_off), 0, 0, 0);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  copy_tile(S0{}, 0);
  if constexpr (NS == 4) {
    copy_tile(S1{}, 1);
    copy_tile(S2{}, 2);
  }

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

  // mp = running max + 8: a logit moves it only when it exceeds mp, and the
  // weights exp2(x - mp) are the usual exp2(x - max) times 2^-8, a factor
  // that cancels in acc / l.
  float acc[QPW][E];
  float mp[QPW], l[QPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    mp[i] = -__builtin_huge_valf();
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
    const uint64_t sel = ballot((s0 <= lim_l) & (sc >= thr_l));
    copy_tile(std::integral_constant<int, (S + NS - 1) % NS>{}, kt + NS - 1);
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
          const bool up = x > mp[i];
          if (ballot(up) != 0u) {
            const float mn = up ? x + 8.f : mp[i];
            const float alpha = exp2f(mp[i] - mn);  // mp = -inf: 0 on an empty state
            l[i] *= alpha;
#pragma unroll
            for (int e = 0; e < E; ++e) acc[i][e] *= alpha;
            mp[i] = mn;
          }
          // bare v_exp_f32: results below 2^-126 flush to 0, which no sum can see
          const float pr = __builtin_amdgcn_exp2f(x - mp[i]);
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
      for (; u != 0u; u &= u - 1u) {
        const int j = __builtin_ctz(u);
        float ka[E], va[E];
        lds_slice<Tag, E>(kl + j * RB, lane, ka);
        lds_slice<Tag, E>(vl + j * RB, lane, va);
        process(j, ka, va);
      }
    }
  };
  // Four tiles per trip: one per slot.
  for (int kt = 0; kt < nkt; kt += NS) {
    tile(S0{}, kt);
    if (kt + 1 >= nkt) break;
    tile(S1{}, kt + 1);
    if constexpr (NS == 4) {
      if (kt + 2 >= nkt) break;
      tile(S2{}, kt + 2);
      if (kt + 3 >= nkt) break;
      tile(S3{}, kt + 3);
    }
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

bool staged_attn_auto(int dtype, int64_t B, int64_t T, int HQ, int DQ, int DV) {
  if (dtype != 0 || T < kStagedMinT || !staged_attn_supported(dtype, HQ, DQ, DV)) return false;
  if (static_cast<int64_t>(HQ) * DQ != 8 * kWave) return false;  // E = 8
  const int64_t blocks = B * (((T + kSTQ - 1) / kSTQ + 1) / 2);
  return 2 * blocks >= device_cus();
}

hipError_t launch_staged_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, float scale, float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  if (!staged_attn_fits(T, ld)) return hipErrorInvalidValue;
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
