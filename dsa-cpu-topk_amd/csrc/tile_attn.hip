// tile_attn.hip -- threshold-masked attention on MFMA tiles, for long rows (gfx950).
//
// Same result as sparse_attn.hip (reference dsa_attention.py:234-324):
//   sel(t,s) = s <= t && scores[t,s] >= thr[t]
//   O[t,h,:] = sum_{s in sel} softmax_s(<Q[t,h],K[s,h]> * scale) V[s,h,:]
// but computed densely over the causal triangle with the selection applied
// as a mask.  When each query selects a large share of a long row (config 4:
// k = 2048 of up to 16384 keys, every 64x64 tile holds selected pairs), the
// per-query gather re-reads 16 MB of K/V rows per query from L2/MALL; here a
// block of 128 queries shares every K/V tile it loads, and both products run
// on MFMA.
//
// Block = 4 waves = 128 consecutive queries of one (batch element, head);
// wave w owns queries t0+32w .. t0+32w+31 (two 16-query MFMA column tiles).
// Key tiles of 64 keys are copied HBM -> LDS by the DMA path
// (buffer_load_dwordx4 ... lds: no registers, no LDS store instructions;
// range-checked, so rows past T read as zeros), K and V both as plain
// [key][d] rows, double-buffered with one barrier per tile.  Rows are
// stored with their 16-byte chunks XOR-swizzled by row so that every LDS
// read pattern below hits distinct banks.
//
// The selection of a wave's 32 x 64 tile comes either from the fp32 score
// rows and thresholds (kSrcScores*: 8 KB per wave and tile, read by every
// head's block) or from a bitmask built once per (query, key) by
// selection_mask_kernel (kSrcMask: 256 bytes per wave and tile; config 4:
// 1.47 -> 1.10 ms for the kernel, 1.37 GB instead of 7.5 GB of L2 misses).
// Either is loaded one tile ahead, behind the next tile's DMA, and the
// barrier waits for the DMA only.
//
// The products are computed transposed, so that no lane exchanges are needed
// between them (16x16x32 MFMA: A[m][k] lane l holds m = l%16, k-slots
// 8(l/16)..+7; B[k][n] lane l holds n = l%16, the same k-slots; D[m][n] lane
// l holds n = l%16, m = 4(l/16)+r):
//   S^T = K . Q^T   A = K rows (LDS), B = Q^T (registers, loaded once)
//                   -> lane l: query l%16, keys 4(l/16)+r of each 16-key tile
//   softmax state (running max m, normaliser l) is per query = per lane
//   O^T = V^T . P^T A = V^T (from the [key][d] V rows by the transposing
//                   LDS read ds_read_b64_tr_b16: within each 16-lane group,
//                   lane i's element s is element i%4 of the 8 bytes lane
//                   4s+i/4 addressed, so lanes addressing rows key0+4g+j/4,
//                   dims 16dt+4(j%4) receive d = 16dt+i, keys key0+4g+s),
//                   B = P^T straight from the S^T registers: the 8 k-slots of
//                   lane group g are keys {4g..4g+3} of key tile 2j and of
//                   key tile 2j+1
//                   -> lane l: query l%16, dims 4(l/16)+r of each 16-dim tile
// P is rounded to the input's 16-bit type for the second product and for
// the softmax normaliser, which sums those 16-bit values with v_dot2 against
// (1, 1) (fp32 accumulation), so numerator and denominator sum the same
// probabilities (the reference uses fp32 probabilities; the difference is
// far inside the 16-bit tolerance); everything else is fp32.  Rows that
// select nothing get 0/0 = NaN, as the reference.
#include <mutex>
#include <type_traits>

#include "dsa_device.h"
#include "dsa_launch.h"

typedef float dsa_f32x4 __attribute__((ext_vector_type(4)));
// Raw buffer loads (the LLVM intrinsics, bound by asm label, so declared
// outside any namespace).  They are typed as float on purpose: this
// toolchain's optimiser narrows the integer-vector forms (and the clang
// builtin __builtin_amdgcn_raw_buffer_load_b128) to a single dword and
// repeats it in every element.  Arguments: resource, byte offset (VGPR),
// SGPR offset, cache policy.
__device__ dsa_f32x4 buffer_load_f32x4(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");
__device__ float buffer_load_f32(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.f32");
typedef float dsa_f32x2 __attribute__((ext_vector_type(2)));
__device__ dsa_f32x2 buffer_load_f32x2(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v2f32");


namespace dsa {
namespace {

constexpr int kTQ = 128;  // queries per block
constexpr int kKT = 64;   // keys per LDS tile
constexpr int kNT = 256;  // threads per block

struct TileArgs {
  const float* scores;
  int64_t ld;
  const float* thr;
  const void* Q;
  const void* K;
  const void* V;
  int64_t B;
  int T;
  int HQ;
  float scale_log2;
  float* out;
  const uint64_t* mask;  // selection bitmask (kSrcMask): [B*T][ldm] words
  int64_t ldm;
};

// Where a block's selection comes from.
constexpr int kSrcScores4 = 0;  // fp32 scores + thresholds, float4 loads (16-byte rows)
constexpr int kSrcScores1 = 1;  // the same, dword loads
constexpr int kSrcMask = 2;     // selection bitmask (selection_mask_kernel)

template <typename Tag>
struct Mfma16x16x32;

template <>
struct Mfma16x16x32<BF16> {
  static __device__ __forceinline__ f32x4 run(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static constexpr uint32_t kOnes = 0x3f803f80u;  // two bf16 1.0
  static __device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {  // acc + w.lo + w.hi
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                           __builtin_bit_cast(bf16x2, kOnes), acc, false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {  // one v_cvt_pk_bf16_f32
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
  }
};

template <>
struct Mfma16x16x32<F16> {
  static __device__ __forceinline__ f32x4 run(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static constexpr uint32_t kOnes = 0x3c003c00u;  // two f16 1.0
  static __device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, kOnes), acc,
                                  false);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define DSA_LDS __attribute__((address_space(3)))

// One K or V tile in LDS: 64 rows of D 16-bit elements, 16-byte chunk c of
// row r stored at chunk position c ^ swz(r).
template <int D>
struct TileLds {
  static constexpr int NCH = D / 8;  // 16-byte chunks per row
  static constexpr int BYTES = kKT * D * 2;
  // K is read as 16-byte A fragments by 16 consecutive rows at one chunk:
  // row % NCH spreads them over NCH chunk positions.
  static __device__ __forceinline__ int swz_k(int r) { return r & (NCH - 1); }
  // V is read by the transposing 8-byte reads: 4 consecutive rows at one
  // chunk pair {2m, 2m+1} per 16-lane group; 2*(r % (NCH/2)) keeps the pair
  // together and moves it per row.
  static __device__ __forceinline__ int swz_v(int r) { return (2 * r) & (NCH - 1); }
};

// Buffer resource over one head's K or V rows from row s1 on (`head_base`
// is row 0 of this batch element at this head's columns): rows_rsrc, whose
// size ends at row T, so DMA reads of rows at or past T return zeros with no
// per-row clamp.  Those rows are never causal for any query, so they are
// masked to -inf and their zero V rows add 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char* head_base, int s1, int T,
                                                          uint32_t rowbytes) {
  return rows_rsrc(head_base, s1, T, rowbytes);
}

// Issue this wave's share of the DMA of one 64-row tile into `dst`: PW
// 1 KiB instructions (buffer_load_dwordx4 ... lds: no registers, no LDS
// store instructions); off[i] is the lane's loop-invariant byte offset of
// its 16-byte chunk within the tile.  Completion is awaited with vmcnt
// before the barrier that publishes the tile.
template <int PW>
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rsrc, const uint32_t (&off)[PW],
                                         DSA_LDS uint8_t* dst, int wave) {
#pragma unroll
  for (int i = 0; i < PW; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst + (wave * PW + i) * 1024, 16,
                                             static_cast<int>(off[i]), 0, 0, 0);
}

// Wait until at most N vector-memory operations of this wave are
// outstanding: the ones issued last (a tile's score loads) may stay in
// flight, everything issued before them (the DMA) has completed.
template <int N>
__device__ __forceinline__ void wait_dma_keep() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <typename Tag, int D, int SRC>
__global__ __launch_bounds__(kNT, 2) void tile_attn_kernel(TileArgs a) {
  static_assert(D == 64 || D == 128, "head dim");
  constexpr bool VEC = SRC == kSrcScores4;
  constexpr bool MASK = SRC == kSrcMask;
  using M = Mfma16x16x32<Tag>;
  using L = TileLds<D>;
  constexpr int NKS = D / 32;  // k-steps of the first product
  constexpr int NDT = D / 16;  // 16-dim output tiles
  // 16-key tiles whose K fragments are read at once (all four unless the
  // prefetched fp32 scores leave too few registers)
  constexpr int KJ = (D == 128 && !MASK) ? 2 : 4;
  constexpr int VG = 4;                 // 16-dim output tiles whose V fragments are read at once
  // Two buffers per operand, as separate objects: the compiler then knows a
  // DMA into one buffer does not alias reads of the other, and keeps the
  // next tile's DMA in flight while the current tile is read.
  __shared__ __align__(16) uint8_t k0[L::BYTES], k1[L::BYTES], v0[L::BYTES], v1[L::BYTES];
  // Bitmask form: the bias of the four keys one nibble of a mask word
  // covers, entry n = {bit r of n set ? 0 : -inf, r = 0..3} (256 bytes).
  // The S accumulators start from it, so an unselected key's logit leaves
  // the MFMA as -inf + logit and a selected one as +0 + logit.  Its larger
  // alignment puts it at LDS address 0, so an entry's address is the nibble
  // times 16 with no base to add (one VALU instruction less per nibble;
  // past the 64 KB of K/V tiles the base does not fit the read's offset).
  __shared__ __align__(1024) float btab[MASK ? 64 : 4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS targets in SGPRs
  const int lane = lane_id();
  const int g = lane >> 4, c16 = lane & 15;
  const int T = a.T;
  const int HQ = a.HQ;
  if constexpr (MASK) {  // published by the barrier before the first tile
    if (tid < 64) btab[tid] = (((tid >> 2) >> (tid & 3)) & 1) ? 0.f : -__builtin_huge_valf();
  }
  const DSA_LDS uint8_t* const btabl = (const DSA_LDS uint8_t*)btab;

  // Block -> (tile, batch, head): tiles longest first, then batch, head fastest.
  const int ntile = (T + kTQ - 1) / kTQ;
  const int64_t per_tile = a.B * HQ;
  const int tile = ntile - 1 - static_cast<int>(blockIdx.x / per_tile);
  const int64_t bh = blockIdx.x % per_tile;
  const int64_t b = bh / HQ;
  const int h = static_cast<int>(bh % HQ);
  const int t0 = tile * kTQ;
  const int tw = t0 + 32 * wave;  // first query of this wave

  const int64_t rowE = static_cast<int64_t>(HQ) * D;  // elements per Q/K/V row
  const uint16_t* Qb = static_cast<const uint16_t*>(a.Q) + b * T * rowE + static_cast<int64_t>(h) * D;
  const uint16_t* Kb = static_cast<const uint16_t*>(a.K) + b * T * rowE + static_cast<int64_t>(h) * D;
  const uint16_t* Vb = static_cast<const uint16_t*>(a.V) + b * T * rowE + static_cast<int64_t>(h) * D;

  const int s_hi = min(T, t0 + kTQ);          // keys [0, s_hi) can be causal in this block
  const int nkt = (s_hi + kKT - 1) / kKT;
  const int wave_last = min(tw + 31, T - 1);  // last query of this wave

  // Loop-invariant DMA offsets of this wave's chunks within a tile: physical
  // chunk P of the tile holds row P / NCH, logical chunk (P % NCH) ^ swz(row).
  constexpr int PW = L::BYTES / 1024 / (kNT / kWave);
  const uint32_t rowbytes = static_cast<uint32_t>(rowE) * 2u;
  uint32_t koff[PW], voff[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int P = (wave * PW + i) * 64 + lane;
    const int r = P / L::NCH, pc = P % L::NCH;
    koff[i] = static_cast<uint32_t>(r) * rowbytes + 16u * static_cast<uint32_t>(pc ^ L::swz_k(r));
    voff[i] = static_cast<uint32_t>(r) * rowbytes + 16u * static_cast<uint32_t>(pc ^ L::swz_v(r));
  }
  const char* const kbase = reinterpret_cast<const char*>(Kb);
  const char* const vbase = reinterpret_cast<const char*>(Vb);
  dma_tile<PW>(tile_rsrc(kbase, 0, T, rowbytes), koff, (DSA_LDS uint8_t*)k0, wave);
  dma_tile<PW>(tile_rsrc(vbase, 0, T, rowbytes), voff, (DSA_LDS uint8_t*)v0, wave);

  // Q^T fragments: qf[qt][ks] = Q[query tw+16qt+c16][dims 32ks+8g .. +8].
  u32x4 qf[2][NKS];
  int tq[2];
  float thr[2];
  uint32_t soff[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    tq[qt] = tw + 16 * qt + c16;
    const int tl = min(tq[qt], T - 1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qf[qt][ks] = *reinterpret_cast<const u32x4*>(Qb + tl * rowE + 32 * ks + 8 * g);
    if constexpr (MASK) {
      thr[qt] = 0.f;
      // byte offset of the query's mask row from row t0 (< 128 rows: the
      // host keeps 128 * ldm * 8 below 2^31)
      soff[qt] = static_cast<uint32_t>(tl - t0) * static_cast<uint32_t>(a.ldm) * 8u;
    } else {
      thr[qt] = a.thr[b * T + tl];
      // byte offset of the query's score row from row t0 (< 128 rows: the
      // host keeps 128 * ld * 4 below 2^31), plus this lane group's 4 keys
      soff[qt] = static_cast<uint32_t>(tl - t0) * static_cast<uint32_t>(a.ld) * 4u + 16u * g;
    }
  }

  float m[2] = {-__builtin_huge_valf(), -__builtin_huge_valf()};
  // Softmax normaliser per query: this lane's part, the sum of the 16-bit
  // probabilities of its 16 keys per tile (the values the O product uses),
  // two at a time by v_dot2 against (1, 1); the query's four lanes are
  // summed at the end.  (Summing with one more MFMA per fragment, ones .
  // P^T, costs 64 MFMA cycles per wave and tile against these 16 VALU
  // instructions: config 4 1.060 ms against 1.035 on one box.)
  float lpart[2] = {0.f, 0.f};
  f32x4 o[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) o[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Per-lane LDS read offsets within a tile (the swizzles depend on the row
  // only through c16 (K) and 4g + c16/4 (V), so they are loop invariant).
  int kofs[NKS], vofs[NDT];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) kofs[ks] = c16 * (2 * D) + 16 * ((4 * ks + g) ^ L::swz_k(c16));
  {
    const int vr = 4 * g + (c16 >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
      vofs[dt] = vr * (2 * D) + 16 * ((2 * dt + ((c16 & 3) >> 1)) ^ L::swz_v(vr)) + 8 * (c16 & 1);
  }

  // This wave's scores of key tile kt: sv[qt][j][r] = scores[tq[qt]][s0 +
  // 16j + 4g + r], by buffer loads against a resource over the block's score
  // rows from key s0 on (uniform), at the lane's invariant row offset plus an
  // immediate per j: no address arithmetic per tile.  The resource ends at
  // the last score of the batch element, so reads past it (keys past T of
  // the last row, never causal) return zeros; keys past T of other rows
  // read the next row, also never causal.  Entries that are not causal are
  // masked in make_sel.
  const char* const sblk =
      MASK ? reinterpret_cast<const char*>(a.mask + (b * T + t0) * a.ldm)
           : reinterpret_cast<const char*>(a.scores + (b * T + t0) * a.ld);
  const uint64_t sbytes = MASK ? static_cast<uint64_t>(T - t0) * static_cast<uint64_t>(a.ldm) * 8u
                               : static_cast<uint64_t>(T - t0) * static_cast<uint64_t>(a.ld) * 4u;
  auto load_scores = [&](int kt, float (&sv)[2][4][4]) __attribute__((always_inline)) {
    const uint64_t s0b = static_cast<uint64_t>(kt) * kKT * 4u;
    const uint64_t rem = sbytes - s0b;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(sblk + s0b), 0, rem > 0xffffffffull ? -1 : static_cast<int>(static_cast<uint32_t>(rem)),
        0x00020000);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int vo = static_cast<int>(soff[qt]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (VEC) {
          const f32x4 f = buffer_load_f32x4(rs, vo + 64 * j, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[qt][j][r] = f[r];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[qt][j][r] = buffer_load_f32(rs, vo + 64 * j + 4 * r, 0, 0);
        }
      }
    }
  };

  // Selection of this wave's 32 x 64 tile: sel[qt][j][r] for (query
  // tq[qt], key s0 + 16j + 4g + r).  Kept as lane masks (one compare each)
  // and applied once per entry in compute, as a select of the logit or
  // -inf -- exact for any logit, NaN and +-inf of unselected keys included
  // (the reference masks them to -inf before its softmax).  Returns whether
  // the wave has work in the tile.  Bitwise & and | keep it branch-free.
  auto make_sel = [&](int kt, const float (&sv)[2][4][4], bool (&sel)[2][4][4]) {
    const int s0 = kt * kKT;
    const bool inner = (s0 + kKT - 1 <= tw) && (tw + 31 < T);  // every entry causal
    bool any = false;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // key s0 + 16j + 4g + r is causal for query tq iff 16j + r <= tq - s0 - 4g:
      // one compare against a constant per entry
      const int dq = (tq[qt] < T) ? tq[qt] - s0 - 4 * g : -1;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // NaN scores and thresholds select nothing
          sel[qt][j][r] = (inner | (16 * j + r <= dq)) & (sv[qt][j][r] >= thr[qt]);
          any |= sel[qt][j][r];
        }
    }
    return s0 <= wave_last && __ballot(any) != 0;
  };

  // Interior tiles (every key below the block's first query, so below T and
  // causal for all its queries): the selection without the causal test.
  // Queries past T (last block of a ragged T) compute values that are never
  // stored; each query's softmax lives in its own column.
  auto make_sel_fast = [&](const float (&sv)[2][4][4], bool (&sel)[2][4][4]) {
    bool any = false;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sel[qt][j][r] = sv[qt][j][r] >= thr[qt];  // NaN selects nothing
          any |= sel[qt][j][r];
        }
    return __ballot(any) != 0;
  };

  // Bitmask source: word kt of each query's mask row (bit i = key 64kt + i
  // selected, causality included), one 8-byte buffer load per query tile,
  // against a resource over the block's mask rows from word kt on.
  auto load_words = [&](int kt, uint64_t (&mw)[2]) __attribute__((always_inline)) {
    const uint64_t w0b = static_cast<uint64_t>(kt) * 8u;
    const uint64_t rem = sbytes - w0b;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(sblk + w0b), 0, rem > 0xffffffffull ? -1 : static_cast<int>(static_cast<uint32_t>(rem)),
        0x00020000);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
      mw[qt] = __builtin_bit_cast(uint64_t, buffer_load_f32x2(rs, static_cast<int>(soff[qt]), 0, 0));
  };
  uint64_t mwc[2] = {0, 0};  // bitmask words of the tile compute() works on
  // Everything one wave does with key tile kt, staged in (kl, vl).
  auto compute = [&](const bool (&sel)[2][4][4], const DSA_LDS uint8_t* kl,
                     const DSA_LDS uint8_t* vl) __attribute__((always_inline)) {
    // S^T = K . Q^T; A fragment = K row 16j+c16, chunk 4ks+g (swizzled):
    // byte offset kofs[ks] + 16j rows (swz_k(16j+c16) = swz_k(c16)).
    // The K fragments of two 16-key tiles are read together before their
    // products (a scheduling fence keeps them together), so one LDS latency
    // is paid per half tile instead of one per fragment.
    f32x4 st[4][2];
    if constexpr (MASK) {
      // entry (j, r) of lane group g is bit 16j + r of the word shifted
      // right by 4g: nibble j of it indexes the bias table
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const uint64_t w = mwc[qt] >> (4 * g);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t h = static_cast<uint32_t>(w >> (32 * (j >> 1)));
          const uint32_t nib = (h >> (16 * (j & 1))) & 15u;
          st[j][qt] = *reinterpret_cast<const DSA_LDS f32x4*>(btabl + 16 * nib);
        }
      }
    }
    // The wave issues its MFMA groups (S here, O below) at raised priority
    // and its softmax at the normal one, so that of the two waves a SIMD
    // holds, the one with MFMAs to issue goes first and the other's VALU work
    // fills in behind them (a wave's own MFMAs and VALU work do not overlap
    // on gfx950; two waves' partly do).  Config 4: 1.040 -> 1.002 ms, the
    // same output; raising it for the normaliser MFMAs as well: 1.014.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int jp = 0; jp < 4; jp += KJ) {
      u32x4 ka[KJ][NKS];
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
          ka[jj][ks] = *reinterpret_cast<const DSA_LDS u32x4*>(kl + kofs[ks] + 16 * (jp + jj) * (2 * D));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj) {
        if constexpr (!MASK) {
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) st[jp + jj][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
          for (int qt = 0; qt < 2; ++qt)
            st[jp + jj][qt] = M::run(ka[jj][ks], qf[qt][ks], st[jp + jj][qt]);
      }
    }

    __builtin_amdgcn_s_setprio(0);
    // Online softmax per query, log2 domain.  The running max moves only
    // when a tile's max exceeds it by more than 2^8 (probabilities stay
    // <= 256, far from overflow in fp32 and exact in scale for 16-bit), so
    // the O rescale is skipped on almost every tile.
    u32x4 pf[2][2];
    bool grow = false;
    float alpha[2];
    // Bitmask form: the entries hold the logit where selected and -inf +
    // logit where not, which is -inf unless the logit is +inf or NaN (a
    // non-finite Q or K row).  The tile max per lane is NaN-propagating
    // (v_maximum3), so such an entry, or a selected NaN logit, shows; the
    // wave then masks its entries exactly (the logit where selected, -inf
    // where not) and takes the max that ignores NaN, as the scores form
    // does.  Without NaN both maxima agree, so either way the result is
    // that of exact masking.
    float mxm[2];
    if constexpr (MASK) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        mxm[qt] = -__builtin_huge_valf();
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) mxm[qt] = __builtin_elementwise_maximum(mxm[qt], st[j][qt][r]);
      }
      if (__ballot(__builtin_isnan(mxm[0]) | __builtin_isnan(mxm[1])) != 0) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              // bit 16j + r of the word shifted right by 4g: a sign-extended
              // bit field (0 or ~0) and a bit select of the logit or -inf.
              // Scalars move between float and integer through
              // __float_as_uint / __uint_as_float: this toolchain
              // miscompiles __builtin_bit_cast of a vector element (every
              // element then reads element 0).
              const uint32_t hw = static_cast<uint32_t>((mwc[qt] >> (4 * g)) >> (32 * (j >> 1)));
              const uint32_t keep =
                  static_cast<uint32_t>(static_cast<int32_t>(hw << (31 - (16 * (j & 1) + r))) >> 31);
              const float x = st[j][qt][r];
              st[j][qt][r] = __uint_as_float((__float_as_uint(x) & keep) | (0xff800000u & ~keep));
            }
          mxm[qt] = -__builtin_huge_valf();
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) mxm[qt] = fmaxf(mxm[qt], st[j][qt][r]);
        }
      }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float mx = -__builtin_huge_valf();
      if constexpr (MASK) {
        mx = mxm[qt];
      } else {
        // masked logits: the logit where selected, -inf where not
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            st[j][qt][r] = sel[qt][j][r] ? st[j][qt][r] : -__builtin_huge_valf();
            mx = fmaxf(mx, st[j][qt][r]);
          }
      }
      // over the 4 lane groups (VALU lane swaps).  mx holds no NaN here (the
      // masked logits' max ignores NaN), so the IEEE maximum gives the same
      // value with no canonicalising instruction per operand, which fmaxf
      // needs on exchanged values: 8 VALU instructions fewer per tile
      // (config 4: 0.970 -> 0.964 ms, the output unchanged).
      {
        const auto r16 =
            __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = __builtin_elementwise_maximum(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
        const auto r32 =
            __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = __builtin_elementwise_maximum(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
      }
      const float m_blk = mx * a.scale_log2;
      const bool up = m_blk > m[qt] + 8.f;
      const float m_new = up ? m_blk : m[qt];
      alpha[qt] = up ? exp2f(m[qt] - m_new) : 1.f;   // m = -inf: alpha = 0 on an empty O
      grow |= up && (m[qt] != -__builtin_huge_valf());
      m[qt] = m_new;
      const float m_use = (m_new == -__builtin_huge_valf()) ? 0.f : m_new;
      float p[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)  // bare v_exp_f32; exp2(-inf) = 0 for unselected keys
          p[j][r] = __builtin_amdgcn_exp2f(fmaf(st[j][qt][r], a.scale_log2, -m_use));
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        pf[qt][jj] = u32x4{M::pack(p[2 * jj][0], p[2 * jj][1]), M::pack(p[2 * jj][2], p[2 * jj][3]),
                           M::pack(p[2 * jj + 1][0], p[2 * jj + 1][1]),
                           M::pack(p[2 * jj + 1][2], p[2 * jj + 1][3])};
    }
    if (__ballot(grow) != 0) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[dt][qt][r] *= alpha[qt];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) lpart[qt] *= alpha[qt];
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) lpart[qt] = M::dot2_ones(pf[qt][jj][e], lpart[qt]);

    // O^T += V^T . P^T.  Lane (g, j=c16) addresses V row key0 + 4g + j/4,
    // dims 16dt + 4(j%4) .. +3; rows key0 + 16 and + 32 keep the swizzle, so
    // byte offset vofs[dt] + (32jj + 16h) rows.
    // The V fragments of VG output tiles are read together before their
    // products (one LDS latency per group, as for K above).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dg = 0; dg < NDT; dg += VG) {
      u32x4 vfrag[VG][2];
#pragma unroll
      for (int d = 0; d < VG; ++d)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const DSA_LDS uint8_t* va = vl + vofs[dg + d] + 32 * jj * (2 * D);
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((DSA_LDS s16x4*)va);
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((DSA_LDS s16x4*)(va + 16 * (2 * D)));
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          vfrag[d][jj] = u32x4{l2.x, l2.y, h2.x, h2.y};
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int d = 0; d < VG; ++d)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) o[dg + d][qt] = M::run(vfrag[d][jj], pf[qt][jj], o[dg + d][qt]);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // Per tile kt (in buffers kt % 2, its scores already in sv): mask, then
  // the DMA of tile kt+1 and the loads of its scores (in that order: the
  // barrier at the end waits for the DMA only, vmcnt(NSL), and the score
  // loads stay in flight across it), then the products.  Tiles below the
  // block's first query (2 * tile of them, an even count) take the interior
  // mask (no causal test); the one or two tiles on the diagonal the general
  // one.
  constexpr int NSL = MASK ? 2 : (VEC ? 8 : 32);  // selection load instructions per tile
  float sv[2][4][4];
  uint64_t mw[2];
  bool sel[2][4][4];
  auto load_sel = [&](int kt) __attribute__((always_inline)) {
    if constexpr (MASK) load_words(kt, mw);
    else load_scores(kt, sv);
  };
  auto step = [&](auto interior, int kt, DSA_LDS uint8_t* kc, DSA_LDS uint8_t* vc,
                  DSA_LDS uint8_t* kn, DSA_LDS uint8_t* vn) __attribute__((always_inline)) {
    bool act;
    if constexpr (MASK) {  // the words are kept: the prefetch below overwrites mw
      act = __ballot((mw[0] | mw[1]) != 0) != 0;
      mwc[0] = mw[0];
      mwc[1] = mw[1];
    }
    else act = decltype(interior)::value ? make_sel_fast(sv, sel) : make_sel(kt, sv, sel);
    const bool more = kt + 1 < nkt;
    if (more) {
      const int s1 = (kt + 1) * kKT;
      dma_tile<PW>(tile_rsrc(kbase, s1, T, rowbytes), koff, kn, wave);
      dma_tile<PW>(tile_rsrc(vbase, s1, T, rowbytes), voff, vn, wave);
      __builtin_amdgcn_sched_barrier(0);  // the DMA is issued before the selection loads
      load_sel(kt + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (act) compute(sel, kc, vc);
    if (more) wait_dma_keep<NSL>();
    else wait_dma_keep<0>();
    block_sync_lds();
  };
  using Interior = std::integral_constant<bool, true>;
  using Diagonal = std::integral_constant<bool, false>;
  DSA_LDS uint8_t* const kl0 = (DSA_LDS uint8_t*)k0;
  DSA_LDS uint8_t* const kl1 = (DSA_LDS uint8_t*)k1;
  DSA_LDS uint8_t* const vl0 = (DSA_LDS uint8_t*)v0;
  DSA_LDS uint8_t* const vl1 = (DSA_LDS uint8_t*)v1;
  __builtin_amdgcn_sched_barrier(0);
  load_sel(0);
  __builtin_amdgcn_sched_barrier(0);
  wait_dma_keep<NSL>();
  block_sync_lds();
  const int nint = 2 * tile;  // < nkt: the block's first query t0 < T
  for (int kt = 0; kt < nint; kt += 2) {
    step(Interior{}, kt, kl0, vl0, kl1, vl1);
    step(Interior{}, kt + 1, kl1, vl1, kl0, vl0);
  }
  step(Diagonal{}, nint, kl0, vl0, kl1, vl1);
  if (nint + 1 < nkt) step(Diagonal{}, nint + 1, kl1, vl1, kl0, vl0);

  // O = O^T / l, lane l: query tq[qt], dims 16dt + 4g .. +3.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    // l == 0 only if nothing passed: NaN, as the reference
    const float inv = 1.f / sum_xor32(sum_xor16(lpart[qt]));
    if (tq[qt] < T) {
      float* orow = a.out + ((b * T + tq[qt]) * HQ + h) * static_cast<int64_t>(D);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const f32x4 v = o[dt][qt];
        *reinterpret_cast<float4*>(orow + 16 * dt + 4 * g) =
            make_float4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
      }
    }
  }
}

template <typename Tag, int D>
hipError_t launch(const TileArgs& a, int src, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.B * a.HQ * ((a.T + kTQ - 1) / kTQ)));
  if (src == kSrcMask)
    hipLaunchKernelGGL((tile_attn_kernel<Tag, D, kSrcMask>), grid, dim3(kNT), 0, stream, a);
  else if (src == kSrcScores4)
    hipLaunchKernelGGL((tile_attn_kernel<Tag, D, kSrcScores4>), grid, dim3(kNT), 0, stream, a);
  else
    hipLaunchKernelGGL((tile_attn_kernel<Tag, D, kSrcScores1>), grid, dim3(kNT), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_any(const TileArgs& a, int dtype, int D, int src, hipStream_t stream) {
  if (dtype == 1) {
    if (D == 64) return launch<BF16, 64>(a, src, stream);
    if (D == 128) return launch<BF16, 128>(a, src, stream);
  } else if (dtype == 2) {
    if (D == 64) return launch<F16, 64>(a, src, stream);
    if (D == 128) return launch<F16, 128>(a, src, stream);
  }
  return hipErrorInvalidValue;
}

// Selection bitmask of rows (b, t): word w holds keys 64w .. 64w+63, bit i
// set iff key 64w + i <= t and scores[b,t,64w+i] >= thr[b*T+t] (a NaN score
// or threshold selects nothing).  Words 0 .. min(W-1, (t|127)/64) of each
// row are written, W = ceil(T/64): every word the tile kernel's block of
// row t reads.  One wave per row, rows longest first; lane i tests key
// 64w + i and the wave's ballot is word w.  Lane u keeps word 64c + u of
// each group c of 64 words, so each group is one coalesced 512-byte store.
__global__ __launch_bounds__(256) void selection_mask_kernel(const float* __restrict__ scores,
                                                             int64_t ld,
                                                             const float* __restrict__ thr,
                                                             int64_t B, int T, int64_t ldm,
                                                             uint64_t* __restrict__ mask) {
  const int lane = lane_id();
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (idx >= B * T) return;  // whole waves
  const int64_t b = idx % B;
  const int t = T - 1 - static_cast<int>(idx / B);
  const int64_t row = b * T + t;
  const float th = thr[row];
  const float* __restrict__ srow = scores + row * ld;
  uint64_t* __restrict__ mrow = mask + row * ldm;
  const int W = (T + 63) / 64;
  const int nw = min(W, ((t | 127) >> 6) + 1);
  constexpr int U = 16;  // loads in flight per lane
  for (int c = 0; c < nw; c += 64) {
    const int nu = min(64, nw - c);
    uint64_t mine = 0;
    for (int u = 0; u < nu; u += U) {
      float v[U];
#pragma unroll
      for (int e = 0; e < U; ++e)  // in the row; read once: nontemporal
        v[e] = __builtin_nontemporal_load(srow + min(64 * (c + u + e) + lane, t));
#pragma unroll
      for (int e = 0; e < U; ++e) {
        const uint64_t bits = __ballot(64 * (c + u + e) + lane <= t && v[e] >= th);
        mine = (lane == u + e) ? bits : mine;
      }
    }
    if (lane < nu) mrow[c + lane] = mine;
  }
}

}  // namespace

bool tile_attn_supported(int dtype, int HQ, int DQ, int DV, const void* Q, const void* K,
                         const void* V) {
  if (dtype != 1 && dtype != 2) return false;
  if (DQ != DV || (DQ != 64 && DQ != 128)) return false;
  if (HQ < 1) return false;
  for (const void* p : {Q, K, V})
    if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0) return false;
  return true;
}

hipError_t launch_tile_attn(const float* scores, int64_t ld, const float* thr, const void* Q,
                            const void* K, const void* V, int dtype, int64_t B, int64_t T, int HQ,
                            int D, float scale, float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const bool vec = (ld % 4 == 0) && ((reinterpret_cast<uintptr_t>(scores) & 15u) == 0);
  const TileArgs a{scores, ld, thr, Q, K, V, B, static_cast<int>(T), HQ,
                   scale * 1.4426950408889634f, out, nullptr, 0};
  return launch_any(a, dtype, D, vec ? kSrcScores4 : kSrcScores1, stream);
}

hipError_t launch_tile_attn_mask(const uint64_t* mask, int64_t ldm, const void* Q, const void* K,
                                 const void* V, int dtype, int64_t B, int64_t T, int HQ, int D,
                                 float scale, float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const TileArgs a{nullptr, 0, nullptr, Q, K, V, B, static_cast<int>(T), HQ,
                   scale * 1.4426950408889634f, out, mask, ldm};
  return launch_any(a, dtype, D, kSrcMask, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of the bitmask path: the bitmask lives in this
// file-scope device array (one copy per GPU, held until the process ends).
// Host code never passes `scratch` itself to a kernel: its address on each
// device comes from hipGetSymbolAddress, looked up once per device with
// that device current, and that pointer is what the kernels get.
// Calls on one GPU share the array: calls that overlap in time on one GPU
// (different streams, different host threads) race.  Nothing in it needs
// clearing: the mask kernel writes every word the attention kernel reads.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint64_t scratch[kScratchWords];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint64_t* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t scratch_words(uint64_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<uint64_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

hipError_t launch_sparse_attn_mask_noalloc(const float* scores, int64_t ld, const float* thr,
                                           const void* Q, const void* K, const void* V, int dtype,
                                           int64_t B, int64_t T, int HQ, int D, float scale,
                                           float* out, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const int64_t ldm = (T + 63) / 64;
  if (B * T * ldm > kScratchWords) return hipErrorInvalidValue;  // the caller checked
  uint64_t* mask = nullptr;
  hipError_t e = scratch_words(&mask);
  if (e != hipSuccess) return e;
  e = launch_selection_mask(scores, ld, thr, B, T, mask, ldm, stream);
  if (e != hipSuccess) return e;
  return launch_tile_attn_mask(mask, ldm, Q, K, V, dtype, B, T, HQ, D, scale, out, stream);
}

hipError_t launch_selection_mask(const float* scores, int64_t ld, const float* thr, int64_t B,
                                 int64_t T, uint64_t* mask, int64_t ldm, hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const int64_t rows = B * T;
  hipLaunchKernelGGL(selection_mask_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256),
                     0, stream, scores, ld, thr, B, static_cast<int>(T), ldm, mask);
  return hipGetLastError();
}

}  // namespace dsa
