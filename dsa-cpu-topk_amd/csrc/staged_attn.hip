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
// queries are spread over the same key range.  Here a block of 16 waves
// takes 64 queries and streams their causal key range once, in tiles of 16
// keys copied HBM/L2 -> LDS by the DMA path (buffer_load ... lds through
// range-checked buffer resources whose base moves with the tile, so a copy
// costs no per-lane address arithmetic; a ring of 4 slots, 3 tiles ahead,
// for rows of 1 KiB, and of 2 slots, 1 tile ahead, for rows of 2 KiB), and
// every wave computes its queries' selected pairs of the tile from LDS.  Per
// key tile a wave reads its 4 queries' scores (one per lane, copied with
// the tile), turns them into a 64-bit selection mask, and walks the keys any
// of its queries selected: it reads the key's K and V slices from LDS once
// and updates each selecting query.
//
// Which 64 queries, and which of their keys, a block takes (staged_attn_plan):
// two 32-query tiles p and ntile-1-p (equal causal work per block), one
// 64-query group, or a chunk of a 64-query group's keys when the batch has
// fewer groups than the GPU has compute units -- the chunks' partial softmax
// sums go to a caller-provided workspace and staged_merge_kernel combines
// them.  What bounds a block (per-block clock traces at config 3): its
// selected (query, key) pairs, about 25 VALU instructions each in one
// dependent chain per pair (8 FMAs, three DPP adds, the max test, exp2, 16
// accumulator FMAs), with the 4 waves a SIMD holds too few to hide the
// chain -- as tile pairs every block takes 370-455 us for its ~16k pairs,
// whether it streams 2080 keys or 4096; a group near the start of the row,
// whose queries select most of their few keys, takes 150-280 us alone.  A
// tile pair gives every block the same pair count; the groups stream fewer
// keys in all; the split spreads the long streams when there are not enough
// blocks.
//
// Measured at config 3 (B=4, T=4096, k=256, HQ=8, D=64, fp32): 0.434-0.44 ms
// as tile pairs against 0.69-0.75 ms for per-query gathers (as groups 0.47,
// split 0.44-0.50); B=8 0.73 ms as groups (0.85 as pairs); B=2 0.24 ms
// split (0.41 as pairs, 0.37 gathers); B=1 0.18 ms split (0.20 gathers).
// The threshold entry point takes this kernel only where it measured faster
// than the gathers (staged_attn_auto).
//
// Lane layout as in attn_tile.h: a K (or V) row is 64*E elements, lane l
// owns [l*E, (l+1)*E); a head spans DQ/E lanes and its logit is a butterfly
// over them.  Softmax is online in the log2 domain with fp32 state; the
// running max moves only when a logit exceeds it by more than 8 (a factor
// 2^8), so the accumulator is rescaled on a few keys per query.  Rows that select
// nothing output NaN (0/0), as the reference.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "dsa_device.h"
#include "dsa_launch.h"

namespace dsa {
namespace {

constexpr int kSTQ = 32;     // queries per tile; a block holds two tiles
constexpr int kSQ = 2 * kSTQ;  // queries per block (a 64-query group when split)
constexpr int kSTW = 16;     // waves per block
constexpr int kSQPW = kSQ / kSTW;

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
  int CK;          // keys per chunk: a group with more causal keys is split
  int q_split;     // first 64-query group with more than CK causal keys
  int nsplit;      // groups q_split .. nq-1 per batch element
  int ncmax;       // chunks of the longest group
  float* part;     // split groups' partial sums [B][nsplit][ncmax][kSQ][row]
  float* part_ml;  // and their (running max + 8, sum) [B][nsplit][ncmax][kSQ][heads][2]
  // Per batch element, in launch order: tile a | tile b << 12 | chunk << 24
  // (32-query tiles a <= b; a == b: one tile).
  uint32_t items[kStagedMaxItems];
};
static_assert(sizeof(StagedArgs) <= 4096, "kernel arguments are limited to 4 KiB");

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
// butterfly is straight-line code.
//
// Block blockIdx.x serves batch element blockIdx.x % B and work item
// items[blockIdx.x / B]: two 32-query tiles a <= b and chunk c of their
// causal keys, keys [c*CK, min(L, (c+1)*CK)) with L = min(T, 32(b+1)).  Wave
// w owns queries 2w, 2w+1 of each tile.  The host forms the items one of two
// ways (staged_attn_plan): tiles p and ntile-1-p in one chunk (every block
// has about the same causal work, T keys x 32 queries, and the short tile's
// keys come with the long tile's stream), or tiles 2m, 2m+1 -- the 64-query
// group m -- with the group's causal keys split into chunks of CK when it
// has more; the chunks of a split group write partial sums that
// staged_merge_kernel combines.
//
// Pipeline: NS LDS slots (ring_slots), each holding one key tile's K rows,
// V rows and the block's scores for it, all copied by DMA.  Iteration kt
// waits for tile kt's copies, passes one barrier (every wave is then done
// with tile kt-1, whose slot is free), issues the copies of tile kt+NS-1
// into that slot and computes tile kt.  Every iteration issues the same
// copies (tiles past the chunk read rows that nobody uses, or zeros past
// row T, into a slot nobody reads), so the wait is one fixed vmcnt: all but
// the copies of the NS-2 tiles issued after tile kt's.  The slots are
// separate LDS objects and the loop is unrolled over them, so the compiler
// sees that a copy into one slot does not alias reads of another and leaves
// the copies in flight.
template <typename Tag, int E, int LPH>
__global__ __launch_bounds__(kSTW * kWave) void staged_attn_kernel(StagedArgs a) {
  constexpr int QPW = kSQPW;
  constexpr int NW = kSTW;               // waves per block
  constexpr int NT = NW * kWave;         // threads per block
  constexpr int KT = tile_keys<Tag, E>();
  static_assert(KT == 16, "16 keys per tile");
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
  constexpr int HQ = kWave / LPH;  // heads per row
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
  const uint32_t item = a.items[static_cast<int64_t>(blockIdx.x) / a.B];
  const int ta = static_cast<int>(item & 0xfffu);
  const int tb = static_cast<int>((item >> 12) & 0xfffu);
  const int chunk = static_cast<int>(item >> 24);
  const int L = min(T, kSTQ * (tb + 1));  // causal keys of the block's last query
  const int k0 = chunk * a.CK;
  const int k1 = min(L, k0 + a.CK);
  const bool split = L > a.CK;  // only for 64-query groups (ta = 2m, tb = 2m+1)
  const int nkt = (k1 - k0 + KT - 1) / KT;
  constexpr int HALF = QPW / 2;  // queries per wave from each tile

  // Query i of this wave: 2*wave + i % 2 of tile ta (i < 2) or of tile tb;
  // its row in a 64-query group's partial sums is (i < 2 ? 0 : 32) + 2*wave
  // + i % 2.
  auto query_of = [&](int i) { return (i < HALF ? ta : tb) * kSTQ + HALF * wave + (i % HALF); };
  auto valid = [&](int i, int t) { return t < T && (i < HALF || tb != ta); };

  // This lane's score per key tile: query lane / KT of the wave, key
  // s0 + lane % KT, clamped into the row (the mask tests causality).  Keys
  // at or past k1 are never causal: k1 is L (past every query of the tile)
  // or a chunk end, where the tile loop stops.
  const int j_l = lane % KT;
  const int i_l = lane / KT;
  const int t_l = (i_l < HALF ? ta : tb) * kSTQ + HALF * wave + (i_l % HALF);
  const bool v_l = t_l < T && (i_l < HALF || tb != ta);
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
    const int s0 = k0 + t * KT;
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
  // that cancels in acc / l (and in the merge of split tiles, which rescales
  // every chunk to the largest mp).
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
    const int s0 = k0 + kt * KT;
    const float sc = *reinterpret_cast<const DSA_LDS float*>(cs[S] + wave * (kWave * 4) + lane * 4);
    // bit i*KT + j: query i of the wave selects key s0 + j (NaN scores and
    // thresholds select nothing)
    const uint64_t sel = ballot((s0 <= lim_l) & (sc >= thr_l));
    // The next tile's copies issue at raised wave priority: they go out
    // before the other waves' pair arithmetic takes the SIMD (config 3:
    // 0.452 -> 0.439 ms, B=2 0.250 -> 0.241; the same output).
    __builtin_amdgcn_s_setprio(1);
    copy_tile(std::integral_constant<int, (S + NS - 1) % NS>{}, kt + NS - 1);
    __builtin_amdgcn_s_setprio(0);
    uint32_t u = static_cast<uint32_t>((sel | (sel >> 16) | (sel >> 32) | (sel >> 48)) & 0xffffu);
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
  // NS tiles per trip: one per slot.
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

  // Slot of this chunk's partial rows (split groups only).
  const int64_t pslot =
      ((b * a.nsplit + (ta / 2 - a.q_split)) * a.ncmax + chunk) * static_cast<int64_t>(kSQ);
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int t = query_of(i);
    if (!valid(i, t)) continue;
    if (!split) {
      const float inv = 1.f / l[i];  // l == 0 only if nothing passed: NaN, as the reference
      float* orow = a.out + (b * T + t) * static_cast<int64_t>(RE) + lane * E;
#pragma unroll
      for (int e = 0; e < E; e += 4)
        *reinterpret_cast<float4*>(orow + e) =
            make_float4(acc[i][e] * inv, acc[i][e + 1] * inv, acc[i][e + 2] * inv,
                        acc[i][e + 3] * inv);
    } else {
      const int64_t r = pslot + (i < HALF ? 0 : kSTQ) + HALF * wave + (i % HALF);
      float* prow = a.part + r * RE + lane * E;
#pragma unroll
      for (int e = 0; e < E; e += 4)
        *reinterpret_cast<float4*>(prow + e) =
            make_float4(acc[i][e], acc[i][e + 1], acc[i][e + 2], acc[i][e + 3]);
      if (lane % LPH == 0)  // every lane of a head holds the head's mp and l
        *reinterpret_cast<float2*>(a.part_ml + (r * HQ + lane / LPH) * 2) = make_float2(mp[i], l[i]);
    }
  }
}

// Output rows of the split tiles from their chunks' partial sums: one wave
// per query.  With M the largest mp of a head over the chunks, the head's
// output is sum_c 2^(mp_c - M) acc_c / sum_c 2^(mp_c - M) l_c (a chunk that
// selected nothing has mp = -inf, l = 0, acc = 0 and weight 0; a row whose
// chunks all selected nothing comes out 0/0 = NaN, as the reference).
struct MergeArgs {
  int64_t B;
  int T;
  int CK;
  int q_split;
  int nsplit;
  int ncmax;
  const float* part;
  const float* part_ml;
  float* out;
};

template <int E, int LPH>
__global__ __launch_bounds__(256) void staged_merge_kernel(MergeArgs a) {
  constexpr int RE = kWave * E;
  constexpr int HQ = kWave / LPH;
  const int lane = lane_id();
  const int64_t gq = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // split query
  const int64_t per_b = static_cast<int64_t>(a.nsplit) * kSQ;
  if (gq >= a.B * per_b) return;
  const int64_t b = gq / per_b;
  const int si = static_cast<int>((gq % per_b) / kSQ);
  const int iq = static_cast<int>(gq % kSQ);
  const int qt = a.q_split + si;
  const int t = qt * kSQ + iq;
  if (t >= a.T) return;
  const int L = min(a.T, kSQ * (qt + 1));
  const int nc = (L + a.CK - 1) / a.CK;
  const int h = lane / LPH;
  const int64_t r0 = ((b * a.nsplit + si) * a.ncmax) * static_cast<int64_t>(kSQ) + iq;
  float M = -__builtin_huge_valf();
  for (int c = 0; c < nc; ++c) M = fmaxf(M, a.part_ml[((r0 + c * kSQ) * HQ + h) * 2]);
  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float lsum = 0.f;
  for (int c = 0; c < nc; ++c) {
    const int64_t r = r0 + c * kSQ;
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + (r * HQ + h) * 2);
    const float w = ml.x == -__builtin_huge_valf() ? 0.f : exp2f(ml.x - M);
    lsum = fmaf(w, ml.y, lsum);
    const float* prow = a.part + r * RE + lane * E;
#pragma unroll
    for (int e = 0; e < E; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(prow + e);
      acc[e] = fmaf(w, v.x, acc[e]);
      acc[e + 1] = fmaf(w, v.y, acc[e + 1]);
      acc[e + 2] = fmaf(w, v.z, acc[e + 2]);
      acc[e + 3] = fmaf(w, v.w, acc[e + 3]);
    }
  }
  const float inv = 1.f / lsum;
  float* orow = a.out + (b * a.T + t) * static_cast<int64_t>(RE) + lane * E;
#pragma unroll
  for (int e = 0; e < E; e += 4)
    *reinterpret_cast<float4*>(orow + e) =
        make_float4(acc[e] * inv, acc[e + 1] * inv, acc[e + 2] * inv, acc[e + 3] * inv);
}

template <typename Tag, int E, int LPH>
hipError_t launch(const StagedArgs& a, int nitems, hipStream_t stream) {
  hipLaunchKernelGGL((staged_attn_kernel<Tag, E, LPH>),
                     dim3(static_cast<unsigned>(a.B * nitems)), dim3(kSTW * kWave), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.nsplit == 0) return e;
  MergeArgs m{a.B, a.T, a.CK, a.q_split, a.nsplit, a.ncmax, a.part, a.part_ml, a.out};
  const int64_t nq = a.B * a.nsplit * kSQ;
  hipLaunchKernelGGL((staged_merge_kernel<E, LPH>), dim3(static_cast<unsigned>((nq + 3) / 4)),
                     dim3(256), 0, stream, m);
  return hipGetLastError();
}

// The work items of one batch element (encoded as StagedArgs::items), in
// launch order.  kStagedPairs: tiles p and ntile-1-p, one chunk, p
// ascending (the longest streams first).  kStagedGroups: the 64-query
// groups, one chunk each, the last (longest) first.  kStagedSplit: the
// groups with their causal keys in chunks of CK, the group nearest the
// start first, then the longest chunk: a query selects a larger share of
// its keys the fewer it has, so the early groups compute the most pairs per
// streamed key; they start first, and the short chunks fill the compute
// units that finish early.  Returns the count, -1 past kStagedMaxItems.
int staged_items(int64_t T, int mode, int CK, uint32_t* items) {
  const int ntile = static_cast<int>((T + kSTQ - 1) / kSTQ);
  auto code = [](int ta, int tb, int c) {
    return static_cast<uint32_t>(ta) | (static_cast<uint32_t>(tb) << 12) |
           (static_cast<uint32_t>(c) << 24);
  };
  const int nq = (ntile + 1) / 2;
  if (mode == kStagedPairs || mode == kStagedGroups) {
    if (nq > kStagedMaxItems) return -1;
    for (int q = 0; q < nq; ++q) {
      const int m = nq - 1 - q;
      items[q] = mode == kStagedPairs ? code(q, ntile - 1 - q, 0)
                                      : code(2 * m, std::min(2 * m + 1, ntile - 1), 0);
    }
    return nq;
  }
  struct It { int m, len, c; };
  std::vector<It> v;
  for (int m = 0; m < nq; ++m) {
    const int L = static_cast<int>(std::min<int64_t>(T, int64_t{kSQ} * (m + 1)));
    for (int c = 0; c * CK < L; ++c) v.push_back({m, std::min(L, (c + 1) * CK) - c * CK, c});
  }
  if (static_cast<int>(v.size()) > kStagedMaxItems || (v.empty() ? 0 : v.back().c) > 255) return -1;
  std::stable_sort(v.begin(), v.end(), [](const It& x, const It& y) {
    if (x.m != y.m) return x.m < y.m;
    if (x.len != y.len) return x.len > y.len;
    return x.c < y.c;
  });
  for (size_t i = 0; i < v.size(); ++i)
    items[i] = code(2 * v[i].m, std::min(2 * v[i].m + 1, ntile - 1), v[i].c);
  return static_cast<int>(v.size());
}

}  // namespace

StagedPlan staged_attn_plan(int64_t B, int64_t T, int HQ, int DQ, bool split) {
  StagedPlan p{};
  const int64_t nq = (T + kSQ - 1) / kSQ;  // 64-query groups
  const int cus = std::max(device_cus(), 1);
  p.CK = 1 << 30;
  // Measured at T = 4096, HQ = 8, D = 64, k = 256 fp32 on MI355X (256 CUs):
  // B = 8 0.73 ms as groups against 0.85 as tile pairs; B = 4 0.44 as tile
  // pairs against 0.44-0.47 as groups, split or not; B = 2 0.238 ms split
  // into chunks of 512 keys (0.248 with 256, 0.41 as tile pairs); B = 1
  // 0.176 ms with chunks of 256 (0.216 with 512, 0.41 as tile pairs).
  if (B * nq >= 2 * cus) {
    p.mode = kStagedGroups;
  } else if (B * nq >= cus || !split) {
    p.mode = kStagedPairs;
  } else {
    // Chunks of half the mean number of keys a unit streams, in multiples
    // of 256.
    int64_t keys = 0;
    for (int64_t m = 0; m < nq; ++m) keys += std::min(T, kSQ * (m + 1));
    int64_t ck = std::max<int64_t>(256, B * keys / cus / 2 / 256 * 256);
    uint32_t tmp[kStagedMaxItems];
    while (ck < T && staged_items(T, kStagedSplit, static_cast<int>(ck), tmp) < 0) ck *= 2;
    if (ck < T) {
      p.mode = kStagedSplit;
      p.CK = static_cast<int>(ck);
    } else {
      p.mode = kStagedPairs;
    }
  }
  if (p.mode != kStagedSplit) return p;  // no group is split: no workspace
  p.q_split = p.CK / kSQ;  // groups m >= CK/64 have more than CK causal keys
  p.nsplit = static_cast<int>(nq - p.q_split);
  p.ncmax = static_cast<int>((T + p.CK - 1) / p.CK);
  const int64_t rows = B * p.nsplit * p.ncmax * kSQ;
  p.part_bytes = rows * HQ * DQ * 4;
  p.ws_bytes = p.part_bytes + rows * HQ * 2 * 4;
  return p;
}

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

bool staged_attn_auto(int dtype, int64_t B, int64_t T, int HQ, int DQ, int DV, bool split) {
  if (dtype != 0 || T < kStagedMinT || !staged_attn_supported(dtype, HQ, DQ, DV)) return false;
  if (static_cast<int64_t>(HQ) * DQ != 8 * kWave) return false;  // E = 8
  if (split) return true;
  const int64_t blocks = B * (((T + kSTQ - 1) / kSTQ + 1) / 2);
  return 2 * blocks >= device_cus();
}

hipError_t launch_staged_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                              const void* K, const void* V, int dtype, int64_t B, int64_t T,
                              int HQ, int DQ, float scale, float* out, void* ws, int64_t ws_bytes,
                              hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  if (!staged_attn_fits(T, ld)) return hipErrorInvalidValue;
  StagedPlan p = staged_attn_plan(B, T, HQ, DQ, true);
  if (p.mode == kStagedSplit && (ws == nullptr || ws_bytes < p.ws_bytes ||
                                 (reinterpret_cast<uintptr_t>(ws) & 15u) != 0))
    p = staged_attn_plan(B, T, HQ, DQ, false);
  StagedArgs a{};
  a.scores = scores; a.ld = ld; a.thr = thr; a.Q = Q; a.K = K; a.V = V; a.B = B;
  a.T = static_cast<int>(T); a.DQ = DQ; a.scale_log2 = scale * 1.4426950408889634f; a.out = out;
  a.CK = p.CK; a.q_split = p.q_split; a.nsplit = p.nsplit; a.ncmax = p.ncmax;
  if (p.nsplit > 0) {
    a.part = static_cast<float*>(ws);
    a.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + p.part_bytes);
  }
  const int nitems = staged_items(T, p.mode, p.CK, a.items);
  if (nitems < 0) return hipErrorInvalidValue;
  const int E = static_cast<int>(static_cast<int64_t>(HQ) * DQ / kWave);
  const int lph = DQ / E;
#define DSA_STAGED_LPH(Tag, e)                                      \
  switch (lph) {                                                    \
    case 1: return launch<Tag, e, 1>(a, nitems, stream);            \
    case 2: return launch<Tag, e, 2>(a, nitems, stream);            \
    case 4: return launch<Tag, e, 4>(a, nitems, stream);            \
    case 8: return launch<Tag, e, 8>(a, nitems, stream);            \
    case 16: return launch<Tag, e, 16>(a, nitems, stream);          \
    case 32: return launch<Tag, e, 32>(a, nitems, stream);          \
    case 64: return launch<Tag, e, 64>(a, nitems, stream);          \
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
