// Device code of the split-K paged decode attention (C-ABI in pda.h):
// kernel templates shared by the translation units that instantiate them
// (pda_decode_f16.hip, pda_decode_bf16.hip, pda_decode_q8.hip,
// pda_decode_gen.hip) and the host side that plans and launches them
// (pda_kernels.hip).
//
// Reference algorithm: python/instinct/backends/metal_kernels.py:18-124
// (pass one _DECODE_BODY, tails _SINGLE_WRITE/_SPLIT_WRITE, merge
// _DECODE_MERGE). The semantics are those of the portable path
// (portable.py:155-205): visible keys are [max(0, len - window), len), pages
// with a negative id are masked.
#ifndef PDA_DECODE_H
#define PDA_DECODE_H

#include <hip/hip_runtime.h>

#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "pda_internal.h"

namespace pda_decode {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr float kLog2e = 1.44269504088896340736f;
// Lazy rescale threshold (log2 units): probabilities stay below 2^8.
constexpr float kSlack = 8.0f;
constexpr int kSplitWaves = 8;                 // waves per split workgroup (but see split_waves)
// K/V steps in flight per wave (see the split kernel): two; one for the
// matrix-core kernels at D >= 256; four for the VALU kernels at D >= 256
// with at most 2 heads per unit.
constexpr int ring_depth(int d, int g, bool q8, bool gen, bool mf) {
  return mf && d >= 256 ? 1 : !mf && !q8 && !gen && d >= 256 && g <= 2 ? 4 : 2;
}

// Waves of a split workgroup: eight (two per SIMD), except the matrix-core
// kernels at D = 512, whose 16 x 512 output accumulators, queries and
// 32 KiB K/V steps need a whole SIMD's registers per wave (accumulators in
// AGPRs): four waves, one per SIMD.
constexpr int split_waves(int d, bool mf) { return mf && d > 256 ? 4 : kSplitWaves; }
constexpr int kNbuf = 2;                       // K/V steps in flight per wave
constexpr int kTablePages = 64;                // page-table entries held per VGPR refill
constexpr int kMaxGroups = 512;                // resident split workgroups (256 CUs x 2)
constexpr int kMaxWaves = kMaxGroups * kSplitWaves;
constexpr int kMaxPairs = kMaxWaves / 2;
constexpr int kSlots = 2 * kMaxWaves;          // partial slots: first and last unit of a wave
constexpr int kMinPagesPerWave = 1;            // default: spread no thinner than this
constexpr int kMaxBatch = 8184;                // per-sequence tables in LDS: (2B + 1) ints
constexpr int kMergeMaxWaves = 16;             // waves per merge workgroup, at most
constexpr int kMergeSlicedMaxGroups = 4096;    // row-sliced merge grids, at most
constexpr int kMergeSlicedRound = 64;          // candidates of a row-sliced merge wave's round

struct Params {
  const f16* q;
  const f16* k;
  const f16* v;
  const int32_t* tables;
  const int32_t* lengths;
  f16* out;
  int32_t* prefix;    // [B + 1] visible pages before each sequence (workspace)
  int32_t* meet;      // [pairs] pages the first wave of each pair took (workspace)
  float2* part_ml;    // [slots][unit_heads] (running max, sum) of cut units
  float* part_o;      // [slots][unit_heads][D] unnormalised outputs of cut units
  const f16* kscale;  // 8-bit K/V: fp16 scale per (row, kv head) of keys,
  const f16* vscale;  //   of values (null for fp16 K/V)
  int64_t scale_page; // scale elements between pages,
  int32_t scale_head; //   between kv heads of one page,
  int32_t scale_row;  //   between rows of one page and kv head
  int64_t arena_pages;
  int64_t page_bytes; // K/V arena: bytes between pages,
  int32_t head_bytes; //   between kv heads of one page,
  int32_t row_bytes;  //   between rows (keys) of one page and kv head
  int32_t batch;
  int32_t table_stride;
  int32_t page_size;
  int32_t hq;
  int32_t hkv;
  int32_t head_dim;   // elements per row (the template's D except for generic kernels)
  int32_t gtot;       // query heads per kv head
  int32_t nhg;        // head groups per kv head (gtot / unit_heads)
  int32_t unit_heads; // query heads of one unit (G, or fewer for matrix-core kernels)
  int32_t window;
  int32_t grid_pairs; // wave pairs of the split kernel's grid
  int32_t min_pages;  // fewest pages per wave before the stream uses fewer pairs
  int32_t fixed;      // 1: each wave of a pair takes a fixed half of the range
  int32_t balance;    // fixed mode: the wave that is behind its partner raises its priority
  int32_t front256;   // fixed mode: the first wave's share of its pair's range, in 256ths
  int32_t ragged;     // 1: page_size is not a multiple of the keys per step
  int32_t local;      // 1: one workgroup per unit, its pieces merged in LDS (no merge pass)
  float scale_log2;   // scale * log2(e)
  float softcap;      // 0 = off
  float cap_in;       // 2 * log2(e) * scale / softcap
  float cap_out;      // softcap * log2(e)
};

constexpr int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Lane geometry of a head_dim. R lanes share one key; each active lane holds
// EPL elements of it as NV chunks of 8 (one 16-byte load each). Chunk c of
// lane r covers elements [c * DC + r * 8, c * DC + r * 8 + 8), DC = D / NV, so
// one load instruction of the wave reads whole 128-byte lines of KPS rows.
//
// 8-bit K/V (Q8): a lane holds 16 consecutive int8 elements [r * 16, r * 16 +
// 16) of its key, one 16-byte load; R = D / 16, and p.v always runs on key
// pairs, the values of one pair loaded as two 8-byte pieces.
//
// Generic kernels (GEN, any even head dim up to 512): D is the head dim
// padded to a power of two; a lane holds 8 elements [r * 8, r * 8 + 8) of its
// key, loaded as four element pairs (four 4-byte loads at 16 bits, four
// 2-byte loads at 8 bits, since rows of an odd number of pairs are not
// 16-byte aligned); pairs at or past the real head dim are not loaded and
// read as zero. p.v runs on FMAs. Odd head dims (ODD): rows are only 2-byte
// aligned (1-byte at 8 bits), so every element is its own load; the element
// past the head dim reloads the last one, whose query element is zero and
// whose output is never written.
//
// Matrix-core kernels (MF; use_mf in pda_kernels.hip picks the groups each
// head dim takes them at): a step is 16 keys; lane l loads key l % 16,
// elements [32 c + 8 (l / 16), + 8) of
// each 32-element chunk c (NV = D / 32 chunks, one 16-byte load each for K
// and for V), the A operand of v_mfma_f32_16x16x32 as it lands. At 8 bits
// (MF and Q8, D a multiple of 64) chunk c = 2 j + h holds elements
// [64 j + 16 (l / 16) + 8 h, + 8) instead, so that one 16-byte load brings
// a lane's int8 elements of two chunks; the queries follow the same order.
template <int D, bool Q8 = false, bool GEN = false, bool MF = false, bool ODD = false>
struct Geom {
  static constexpr int EPL =
      MF ? D / 4 : GEN ? 8 : Q8 ? 16 : ((D >= 80 && D % 16 == 0) ? 16 : 8);  // per lane
  static constexpr int NV = MF ? D / 32 : (Q8 || GEN) ? 1 : EPL / 8;      // 16-byte K loads
  static constexpr int DC = D / NV;                               // chunk stride
  static constexpr int SLICES = D / EPL;
  static constexpr int R = MF ? 4 : next_pow2(SLICES);            // lanes per key
  static constexpr int KPS = 64 / R;                              // keys per step
  // p.v on v_dot2 over key pairs (head dims with 2R lanes x 8 elements):
  // lane (kp, r2), kp = lane / 2R, r2 = lane % 2R, holds elements
  // [r2 * 8, r2 * 8 + 8) of the step's keys 2 kp and 2 kp + 1.
  static constexpr bool PV2 = !GEN && !MF && EPL == 16 && D == 2 * R * 8;
  static constexpr int OPL = PV2 ? 8 : EPL;                       // outputs per lane
  static constexpr int NPAIR = KPS / 2;                           // key pairs per step
  // Vector memory loads per step: K and V (fp16); K, the two V pieces and the
  // key scale and the pair's two value scales (8-bit); generic: four pieces
  // of K and of V, plus the key's two scales at 8 bits.
  // Matrix-core kernels at 8 bits: NV / 2 pieces of K and of V, the key's
  // two scales. Odd head dims (ODD, generic only): every element on its own,
  // eight of K and eight of V, plus the two scales at 8 bits.
  static constexpr int LOADS = MF ? (Q8 ? NV + 2 : 2 * NV)
                               : GEN ? (ODD ? (Q8 ? 18 : 16) : (Q8 ? 10 : 8))
                               : Q8 ? 6 : 2 * NV;
  static_assert(!ODD || GEN, "odd head dims run the generic kernels");
  static_assert(!MF || (D % 32 == 0 && !GEN && (!Q8 || D % 64 == 0)),
                "matrix-core kernels: D % 32 == 0 (8-bit: D % 64 == 0), no generic dims");
  static_assert(D % EPL == 0 && DC % 8 == 0, "head_dim must be a multiple of 8");
  static_assert(GEN || MF || !Q8 || PV2, "8-bit K/V needs the key-pair p.v layout");
  static_assert(!GEN || (D >= 8 && D <= 512 && (D & (D - 1)) == 0),
                "generic kernels pad the head dim to a power of two");
  static_assert(R <= 64, "head_dim too large");
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                         0xF, 0xF, false));
}

// Sum over the R consecutive lanes that share a key (xor butterfly: every
// lane of the group ends with the bitwise-identical total).
template <int R>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (R >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (R >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (R >= 8) x += dpp<0x141>(x);  // row_half_mirror
  if constexpr (R >= 16) x += dpp<0x140>(x); // row_mirror
  if constexpr (R >= 32) x += __shfl_xor(x, 16);
  if constexpr (R >= 64) x += __shfl_xor(x, 32);
  return x;
}

// Sum over the 64 / R key subsets (lanes r, r + R, r + 2R, ...).
template <int R>
__device__ __forceinline__ float subset_sum(float x) {
  if constexpr (R <= 1) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2] == lane ^ 1
  if constexpr (R <= 2) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1] == lane ^ 2
  if constexpr (R <= 4) x += __shfl_xor(x, 4);
  if constexpr (R <= 8) x += dpp<0x128>(x);  // row_ror:8 == lane ^ 8
  if constexpr (R <= 16) x += __shfl_xor(x, 16);
  if constexpr (R <= 32) x += __shfl_xor(x, 32);
  return x;
}

// Sum over the key pairs of the p.v layout (lanes r2, r2 + 2R, ...).
template <int R>
__device__ __forceinline__ float pair_sum(float x) {
  if constexpr (2 * R <= 8) x += dpp<0x128>(x);  // row_ror:8 == lane ^ 8
  if constexpr (2 * R <= 16) x += __shfl_xor(x, 16);
  if constexpr (2 * R <= 32) x += __shfl_xor(x, 32);
  return x;
}

// The value of lane ^ R (the other key of this lane's pair).
template <int R>
__device__ __forceinline__ float pair_swap(float x) {
  if constexpr (R == 8)  // row_ror:8 == lane ^ 8, every lane valid: no old value
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x128, 0xF, 0xF, true));
  else
    return __shfl_xor(x, R);
}

// a.x * b.x + a.y * b.y in fp32: the 3-operand v_dot2 with an inline zero
// (the compiler would otherwise zero a register to use the accumulating form).
__device__ __forceinline__ float dot2_first(f16x2 a, f16x2 b) {
  float d;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
  return d;
}

// bf16 counterpart of dot2_first.
__device__ __forceinline__ float dot2_first_bf16(bf16x2 a, bf16x2 b) {
  float d;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
  return d;
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Log-sum-exp combination of pieces (metal_kernels.py:103-124): a running
// maximum, pieces whose max is -inf (no visible key) weigh 0.
template <int NC>
__device__ __forceinline__ void lse_add(float& top, float& sum, float (&acc)[NC], float2 ml,
                                        const float (&part)[NC]) {
  if (ml.x == -INFINITY) return;
  const float mn = fmaxf(top, ml.x);
  const float fo = __builtin_amdgcn_exp2f(top - mn);  // 0 while top = -inf
  const float fn = __builtin_amdgcn_exp2f(ml.x - mn);
  top = mn;
  sum = sum * fo + ml.y * fn;
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = acc[c] * fo + part[c] * fn;
}

// s_waitcnt on the vector memory counter alone: at most N loads outstanding
// (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ f16x8 zero_unless(f16x8 x, bool keep) {
  i32x4 bits = __builtin_bit_cast(i32x4, x);
  bits.x = keep ? bits.x : 0;
  bits.y = keep ? bits.y : 0;
  bits.z = keep ? bits.z : 0;
  bits.w = keep ? bits.w : 0;
  return __builtin_bit_cast(f16x8, bits);
}

// Int8 bytes to fp16 pairs, exactly (pda_internal.h).
using pda_internal::bytes_to_f16x2;

// Matrix-core helpers. LDS row of a V tile (16-bit elements): the head dim
// plus padding that puts the four rows one transposed read touches on
// different banks.
constexpr int mf_vrow(int d) { return d % 64 == 32 ? d + 64 : d + 32; }

// S^T += K Q^T over 32 elements: A = 16 keys x 32, B = 32 x 16 heads.
template <bool BF>
__device__ __forceinline__ f32x4 mfma_k32(const f16x8& a, const f16x8& b, const f32x4& c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// O^T += V^T P^T over 16 keys: A = 16 elements x 16 keys, B = 16 keys x 16 heads.
template <bool BF>
__device__ __forceinline__ f32x4 mfma_k16(const f16x4& a, const f16x4& b, const f32x4& c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// gfx950 transposing LDS read: in each group of 16 lanes, lane s names four
// 16-bit elements (row s / 4, columns 4 (s % 4) ..) of a 4 x 16 block and
// receives column s of it, rows 0..3.
__device__ __forceinline__ f16x4 read_tr(const f16* at) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)at));
}

struct SeqGeometry {
  int len, first, first_page, npages;
};

// Visible range [first, len) of sequence b (metal_kernels.py:32-36, length
// clamped to the table) and the pages it touches.
__device__ __forceinline__ SeqGeometry sequence_geometry(const Params& p, int b) {
  SeqGeometry g;
  const int P = p.page_size;
  g.len = min(max(p.lengths[b], 0), p.table_stride * P);
  g.first = p.window > 0 ? max(0, g.len - p.window) : 0;
  g.first_page = g.first / P;
  g.npages = g.len > g.first ? (g.len - 1) / P - g.first_page + 1 : 0;
  return g;
}

// Local mode: ints of dynamic LDS before the pieces (the prefix and the
// lengths, 2 B + 1 ints), rounded to 16 bytes.
__host__ __device__ constexpr int local_lds_offset(int batch) { return (2 * batch + 1 + 3) & ~3; }

// Wave pairs the stream of `total` pages is spread over (both kernels agree).
__device__ __forceinline__ int stream_pairs(int64_t total, const Params& p) {
  if (total <= 0) return 0;
  const int64_t want = (total + 2 * p.min_pages - 1) / (2 * p.min_pages);
  return (int)min<int64_t>(want, p.grid_pairs);
}

// Fixed split points: pages of a pair's range of n pages that its first
// wave takes (both kernels agree).
__device__ __forceinline__ int fixed_front(int64_t n, const Params& p) {
  return (int)(n * p.front256 >> 8);
}

// First page of pair q's range, and the pair whose range holds page x.
__device__ __forceinline__ int64_t range_start(int q, int64_t total, int pairs) {
  return (int64_t)q * total / pairs;
}
__device__ __forceinline__ int pair_of(int64_t x, int64_t total, int pairs) {
  return (int)(((x + 1) * pairs - 1) / total);
}

// Exclusive prefix of visible pages over the batch, into LDS (all threads of
// the workgroup), plus each sequence's clamped length.
template <int kThreads>
__device__ void build_prefix(const Params& p, int* s_prefix, int* s_len) {
  constexpr int kWaves = kThreads / 64;
  __shared__ int s_wsum[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int B = p.batch;
  int carry = 0;
  for (int base = 0; base < B; base += kThreads) {
    const int b = base + tid;
    int x = 0;
    if (b < B) {
      const SeqGeometry g = sequence_geometry(p, b);
      x = g.npages;
      s_len[b] = g.len;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off);
      if (lane >= off) x += y;
    }
    if (lane == 63) s_wsum[w] = x;
    __syncthreads();
    int before = carry, block = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      before += i < w ? s_wsum[i] : 0;
      block += s_wsum[i];
    }
    if (b < B) s_prefix[b + 1] = before + x;
    carry += block;
    __syncthreads();
  }
  if (tid == 0) s_prefix[0] = 0;
  __syncthreads();
}

// Split kernel: a persistent grid of wave pairs (see the file comment).
// At least two waves per SIMD (<= 256 registers): with G = 7 or 8 heads the
// few values that do not fit live outside the main loop.
// BF: queries, K/V and output in bf16 (the model dtype of the reference's
// bf16 models; their arenas hold the model dtype, paged_kv.py:156-292). The
// 16-bit buffers are addressed as fp16 storage and reinterpreted: q.k and
// p.v run on bf16 v_dot2, the probabilities are rounded to bf16 for p.v.
// GEN: generic kernel for a head dim p.head_dim below the padded D (Geom).
// MF: matrix-core kernel for a GQA group of 5 to 16 query heads per unit
// (G = 16 slots, p.unit_heads real heads; see mf_step).
// ODD: generic kernel for an odd head dim (paged_decode_odd_kernel).
template <int D, int G, bool Q8, bool BF, bool GEN, bool MF, bool ODD>
__device__ __forceinline__ void split_body(const Params p) {
  constexpr int kWaves = split_waves(D, MF);  // waves of this workgroup
  constexpr int kThreads = 64 * kWaves;
  constexpr int kWgPairs = kWaves / 2;
  // Arithmetic in bf16 (bf16 K/V). Over 8-bit K/V, BF means bf16 queries
  // and output with the fp16 arithmetic of the 8-bit kernels (see qscale).
  constexpr bool BFM = BF && !Q8;
  static_assert(!MF || G == 16, "matrix-core kernels lay 16 head slots out");
  using Gm = Geom<D, Q8, GEN, MF, ODD>;
  constexpr int EPL = Gm::EPL, NV = Gm::NV, DC = Gm::DC, R = Gm::R, KPS = Gm::KPS;
  constexpr bool PV2 = Gm::PV2;
  constexpr int OPL = Gm::OPL;
  // Steps in flight per wave: two; one where a step alone is 16 KiB or more
  // of K and V per wave (matrix-core kernels at D >= 256), which also keeps
  // those kernels within their registers; four at D >= 256 with at most 2 heads per
  // unit, whose small per-step math leaves registers free (config 4's
  // Gemma-style shape, 42.5 -> 39.7 us; depths 3 and 4 were slower on the
  // other configurations).
  constexpr int NBUF = ring_depth(D, G, Q8, GEN, MF);
  extern __shared__ __align__(16) int s_dyn[];
  __shared__ int s_ticket[kWgPairs];
  __shared__ int s_prog[kWaves];  // fixed mode: pages each wave has started
  // Matrix-core kernels: each wave's V tile of one step, [16 keys][kVRow].
  constexpr int kVRow = mf_vrow(D);
  __shared__ __align__(16) f16 s_vt[MF ? kWaves * 16 * kVRow : 1];
  const int B = p.batch;
  int* const s_prefix = s_dyn;         // [B + 1]
  int* const s_len = s_dyn + B + 1;    // [B]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int kk = lane / R;  // key of the step this lane works on
  const int r = lane % R;   // slice of the head this lane holds
  const bool active = r < Gm::SLICES;
  const int d0 = active ? r * 8 : 0;  // first element of chunk 0
  const int r2 = lane % (2 * R);      // p.v layout: element group and key pair
  const int kp = lane / (2 * R);
  const bool hi = kk & 1;             // this lane's key is the second of its pair
  // Key this lane loads within a step (matrix-core kernels: key lane % 16;
  // its 16-lane group lane / 16 picks the elements) and the head it scores.
  const int lk = MF ? (lane & 15) : kk;
  const int mg = lane >> 4;
  // v_perm selectors that pair V elements as (this lane's key, the other),
  // the order of the probability pair below: bytes 0-3 of the source pair
  // are the second key's dword, 4-7 the first key's.
  const uint32_t sel_lo = hi ? 0x05040100u : 0x01000504u;
  const uint32_t sel_hi = hi ? 0x07060302u : 0x03020706u;
  // 8-bit: bytes (this lane's key, the other) of two elements, from the
  // first key's dword (source bytes 4-7) and the second's (0-3).
  const uint32_t sel8_lo = hi ? 0x05010400u : 0x01050004u;
  const uint32_t sel8_hi = hi ? 0x07030602u : 0x03070206u;
  const int P = p.page_size;
  const int spp = (P + KPS - 1) / KPS;  // steps per page (the last one partial if ragged)
  const int nkvg = p.hkv * p.nhg;
  // Row length in elements: D, or the real head dim of a generic kernel.
  const int hd = GEN ? p.head_dim : D;
  constexpr int kElem = Q8 ? 1 : 2;  // bytes per K/V element

  // Local mode: the unit of this workgroup. The p.nhg units of one kv head
  // (head groups reading the same K/V) go to one XCD (workgroups go round
  // robin over the 8 XCDs), so that the XCD's L2 serves their reads.
  int lx = blockIdx.x;
  if (p.local && p.nhg > 1) {
    const int full = (int)(gridDim.x / p.nhg) / 8 * 8;
    if (lx < full * p.nhg) {
      const int xc = lx % 8, j = lx / 8;
      lx = ((j / p.nhg) * 8 + xc) * p.nhg + j % p.nhg;
    }
  }
  if (tid < kWgPairs) s_ticket[tid] = 0;
  if (tid < kWaves) s_prog[tid] = 0;
  build_prefix<kThreads>(p, s_prefix, s_len);  // ends with a barrier
  if (blockIdx.x == 0)
    for (int i = tid; i <= B; i += kThreads) p.prefix[i] = s_prefix[i];
  // Sequences with no visible key get zeros (metal_kernels.py:88-90 with a
  // zero sum); workgroup j takes sequences j, j + grid, ...
  for (int bz = blockIdx.x; bz < B; bz += gridDim.x) {
    if (s_prefix[bz + 1] != s_prefix[bz]) continue;
    f16* const dz = p.out + (int64_t)bz * p.hq * hd;
    if constexpr (ODD) {  // rows of an odd number of elements: 2-byte stores
      for (int i = tid; i < p.hq * hd; i += kThreads) dz[i] = (f16)0.0f;
    } else if constexpr (GEN) {  // rows of an odd number of pairs: 4-byte stores
      for (int i = tid * 2; i < p.hq * hd; i += kThreads * 2)
        *reinterpret_cast<uint32_t*>(dz + i) = 0u;
    } else {
      for (int i = tid * 8; i < p.hq * D; i += kThreads * 8)
        *reinterpret_cast<f16x8*>(dz + i) = f16x8{};
    }
  }
  const int64_t total = (int64_t)s_prefix[B] * nkvg;
  const int npairs = stream_pairs(total, p);
  const int pl = w % kWgPairs;
  const bool back = w >= kWgPairs;  // takes its pair's range from the end
  const int pair = blockIdx.x * kWgPairs + pl;
  // Local mode (short calls): workgroup j serves unit j alone, its pages
  // split evenly over the workgroup's pairs; the pieces go to LDS and the
  // workgroup merges them after its last wave is done (no merge pass).
  // Every wave reaches that barrier: a pair with no pages starts at the
  // unit's first page and takes none.
  const int hpu_k = MF ? p.unit_heads : G;  // heads of a unit
  float* const s_lo = reinterpret_cast<float*>(s_dyn + local_lds_offset(B));  // [waves][hpu][D]
  float2* const s_lml = reinterpret_cast<float2*>(s_lo + kWaves * hpu_k * D);  // [waves][hpu]
  int64_t x0;
  int n_range;
  if (p.local) {
    const int ub = lx / nkvg;
    const int unpg = s_prefix[ub + 1] - s_prefix[ub];
    if (unpg == 0) return;  // the whole workgroup: zeroed above
    const int64_t us = (int64_t)s_prefix[ub] * nkvg + (int64_t)(lx - ub * nkvg) * unpg;
    x0 = us + (int64_t)unpg * pl / kWgPairs;
    n_range = (int)(us + (int64_t)unpg * (pl + 1) / kWgPairs - x0);
    if (lane < hpu_k) s_lml[w * hpu_k + lane] = make_float2(-INFINITY, 0.0f);
  } else {
    if (pair >= npairs) return;
    x0 = range_start(pair, total, npairs);
    n_range = (int)(range_start(pair + 1, total, npairs) - x0);
  }
  const int dir = back ? -1 : 1;
  const int64_t vw = 2 * (int64_t)pair + (back ? 1 : 0);  // slots 2 vw, 2 vw + 1

  // One ticket per page; a ticket below n_range is a page of the range. All
  // lanes take part without a branch, lane 0 adding 1 and the others 0, so
  // lane 0 always reads the count before its own add. The result stays in a
  // VGPR until it is needed, one page later.
  // Fixed mode (p.fixed): no race. The first wave takes the first
  // n_range / 2 pages and the second the rest, counting its own tickets, so
  // where units are cut, and with it every output bit, depends on the
  // inputs and the grid only (the reference's split ranges are fixed too,
  // metal_kernels.py:32-36). The shared counter is still bumped by 0.
  //
  // The SIMD's issue arbiter favours the older wave of a pair, so with fixed
  // halves one wave would finish early and idle. With p.balance the waves
  // publish the pages they have started in LDS, and at each page the wave
  // that is behind its partner (in fractions of their halves, as seen one
  // page earlier) raises its issue priority (s_setprio 1), the other lowers
  // it; this moves only timing, never a cut point.
  const int front_pages = fixed_front(n_range, p);
  const int quota = p.fixed ? (back ? n_range - front_pages : front_pages) : n_range;
  const int partner_quota = n_range - quota;
  const int partner = back ? w - kWgPairs : w + kWgPairs;
  int own_tickets = 0;
  int seen = 0;  // the partner's pages, read at the previous ticket
  auto take_ticket = [&]() -> int {
    const int shared = __hip_atomic_fetch_add(&s_ticket[pl], (lane == 0 && !p.fixed) ? 1 : 0,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int own = own_tickets++;
    // (Four-wave workgroups run one wave per SIMD: no arbiter to steer.)
    if (kWaves == 8 && p.fixed && p.balance) {
      if ((int64_t)own * partner_quota < (int64_t)uniform(seen) * quota)
        __builtin_amdgcn_s_setprio(1);
      else
        __builtin_amdgcn_s_setprio(0);
      __hip_atomic_fetch_add(&s_prog[w], lane == 0 ? 1 : 0, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
      seen = __hip_atomic_load(&s_prog[partner], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return p.fixed ? own : shared;
  };
  auto granted = [&](int t) -> bool { return uniform(t) < quota; };

  // Unit holding the first page this wave would take: the last b with
  // nkvg * prefix[b] <= x (never an empty sequence, since x < total).
  const int64_t xs = back && n_range > 0 ? x0 + n_range - 1 : x0;
  int b = 0;
  {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)s_prefix[mid] * nkvg <= xs) lo = mid; else hi = mid - 1;
    }
    b = lo;
  }
  int npg = s_prefix[b + 1] - s_prefix[b];
  if (npg <= 0) return;  // cannot happen for xs < total; guards the division
  int kvg, pa;
  {
    const int64_t rel = xs - (int64_t)s_prefix[b] * nkvg;
    kvg = (int)(rel / npg);
    pa = (int)(rel - (int64_t)kvg * npg);
  }

  const char* const kbase = reinterpret_cast<const char*>(p.k);
  const char* const vbase = reinterpret_cast<const char*>(p.v);

  bool first_unit = true;
  int taken = 0;               // pages this wave processed
  bool pending = granted(take_ticket());  // the next page along the wave's way is ours

  while (pending) {
    // Unit (b, kvg): pages pa, pa + dir, ... while tickets last.
    const int len = s_len[b];
    const int first = p.window > 0 ? max(0, len - p.window) : 0;
    const int first_page = first / P;
    const int kvh = kvg / p.nhg;
    const int hpu = MF ? p.unit_heads : G;  // query heads of the unit
    const int h0 = kvh * p.gtot + (kvg - kvh * p.nhg) * hpu;
    const int32_t* const table = p.tables + (int64_t)b * p.table_stride + first_page;

    // Queries of the G heads, this lane's slice, as fp16 pairs for v_dot2
    // (bf16: the same bits, read as bf16 pairs where used).
    f16x2 q[MF ? 1 : G][MF ? 1 : EPL / 2];
    // Matrix-core kernels: Q^T as the B operand of S^T = K Q^T, head
    // lane % 16 (zero past the unit's heads), the elements this lane's K
    // loads hold.
    f16x8 qb[MF ? NV : 1];
    // Matrix-core kernels: the first of the 8 elements of a row that chunk c
    // of this lane's K and V loads holds (8-bit: two chunks per load).
    auto mf_elem = [&](int c) {
      return Q8 ? 64 * (c >> 1) + 16 * mg + 8 * (c & 1) : 32 * c + 8 * mg;
    };
    if constexpr (MF) {
      const bool real = (lane & 15) < hpu;
      const f16* qp = p.q + ((int64_t)b * p.hq + h0 + (real ? (lane & 15) : 0)) * D;
#pragma unroll
      for (int c = 0; c < NV; ++c)
        qb[c] = zero_unless(*reinterpret_cast<const f16x8*>(qp + mf_elem(c)), real);
    }
#pragma unroll
    for (int g = 0; g < (MF ? 0 : G); ++g) {
      if constexpr (GEN) {
        // Element pairs d0 + 2i below the real head dim; the rest stay zero,
        // so whatever the K loads of those pairs hold adds nothing.
        const f16* qp = p.q + ((int64_t)b * p.hq + h0 + g) * hd;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = d0 + 2 * i;
          if constexpr (ODD)  // 2-byte aligned rows: one element at a time
            q[g][i] = f16x2{e < hd ? qp[e] : (f16)0.0f, e + 1 < hd ? qp[e + 1] : (f16)0.0f};
          else
            q[g][i] = e < hd ? *reinterpret_cast<const f16x2*>(qp + e) : f16x2{};
        }
      } else if constexpr (Q8) {
        // Elements [r * 16, r * 16 + 16), the slice of the int8 key row.
        const f16* qp = p.q + ((int64_t)b * p.hq + h0 + g) * D + r * 16;
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          const f16x8 xq = *reinterpret_cast<const f16x8*>(qp + 8 * v);
#pragma unroll
          for (int i = 0; i < 4; ++i) q[g][4 * v + i] = f16x2{xq[2 * i], xq[2 * i + 1]};
        }
      } else {
        const f16* qp = p.q + ((int64_t)b * p.hq + h0 + g) * D + d0;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          f16x8 xq = zero_unless(*reinterpret_cast<const f16x8*>(qp + DC * v), active);
#pragma unroll
          for (int i = 0; i < 4; ++i) q[g][4 * v + i] = f16x2{xq[2 * i], xq[2 * i + 1]};
        }
      }
    }

    // bf16 queries over 8-bit K/V (a bf16 model's 8-bit cache): the int8
    // keys are exact in fp16, so the queries go to fp16 as well, scaled by a
    // power of two chosen per unit that puts the largest in [2^14, 2^15).
    // Every bf16 value (8 significant bits) then converts exactly, unless it
    // is more than 2^31 times smaller than the largest (below 2^-17 after
    // scaling, where fp16 subnormals hold fewer than 8 bits), and each score is
    // multiplied back by the same power of two (qscale, folded into the key
    // scale), which is exact. The rest runs as for fp16 queries; only the
    // output is rounded to bf16. (Converting bf16 to fp16 unscaled would
    // overflow past 65504 and lose the low bits below 2^-14.)
    float qscale = 1.0f;
    if constexpr (Q8 && BF) {
      auto wide = [](f16 h) {
        return __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
      };
      float big = 0.0f;
#pragma unroll
      for (int c = 0; c < (MF ? NV : 0); ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) big = fmaxf(big, fabsf(wide(qb[c][i])));
#pragma unroll
      for (int g = 0; g < (MF ? 0 : G); ++g)
#pragma unroll
        for (int i = 0; i < EPL / 2; ++i)
          big = fmaxf(big, fmaxf(fabsf(wide(q[g][i][0])), fabsf(wide(q[g][i][1]))));
      big = wave_max(big);
      int ex = 0;
      if (big > 0.0f && big < INFINITY) ex = __builtin_amdgcn_frexp_expf(big) - 15;
      qscale = __builtin_ldexpf(1.0f, ex);
      const float down = __builtin_ldexpf(1.0f, -ex);
#pragma unroll
      for (int c = 0; c < (MF ? NV : 0); ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) qb[c][i] = (f16)(wide(qb[c][i]) * down);
#pragma unroll
      for (int g = 0; g < (MF ? 0 : G); ++g)
#pragma unroll
        for (int i = 0; i < EPL / 2; ++i)
          q[g][i] = f16x2{(f16)(wide(q[g][i][0]) * down), (f16)(wide(q[g][i][1]) * down)};
    }

    // Matrix-core kernels keep one (max, sum) per lane, for head lane % 16,
    // and O^T in accumulators ob (see mf_step); the others per head.
    constexpr int kHeads = MF ? 1 : G;
    float o[kHeads][MF ? 1 : OPL];
    float l[kHeads];
    float m[kHeads];
    f32x4 ob[MF ? D / 16 : 1];
#pragma unroll
    for (int g = 0; g < kHeads; ++g) {
      l[g] = 0.0f;
      m[g] = -INFINITY;
#pragma unroll
      for (int i = 0; i < (MF ? 1 : OPL); ++i) o[g][i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < (MF ? D / 16 : 1); ++i) ob[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Addressing: a wave-uniform byte offset per step (page and first key of
    // the step) plus 32-bit per-lane offsets: K by (key, kv head, chunk), V
    // by (key pair, kv head, element group) on the p.v path, else as K.
    const uint32_t lane_off =
        MF    ? (uint32_t)(lk * p.row_bytes + kvh * p.head_bytes + 16 * mg)
        : GEN ? (uint32_t)(kk * p.row_bytes + kvh * p.head_bytes)
        : Q8  ? (uint32_t)(kk * p.row_bytes + kvh * p.head_bytes + r * 16)
              : (uint32_t)(kk * p.row_bytes + kvh * p.head_bytes + d0 * 2);
    const uint32_t v_off =
        (GEN || MF) ? lane_off
        : Q8  ? (uint32_t)(2 * kp * p.row_bytes + kvh * p.head_bytes + r2 * 8)
        : PV2 ? (uint32_t)(2 * kp * p.row_bytes + kvh * p.head_bytes + r2 * 16)
              : lane_off;
    // 8-bit scales, in elements from the step's first key: this lane's key,
    // and its pair's keys with this lane's own key first (generic kernels:
    // this lane's key for both).
    const uint32_t ks_off = (uint32_t)(kvh * p.scale_head + lk * p.scale_row);
    const uint32_t vs_own =
        (GEN || MF) ? ks_off
                    : (uint32_t)(kvh * p.scale_head + (2 * kp + (hi ? 1 : 0)) * p.scale_row);
    const uint32_t vs_other = (uint32_t)(kvh * p.scale_head + (2 * kp + (hi ? 0 : 1)) * p.scale_row);
    // Generic kernels: byte offsets of this lane's four element pairs in a
    // row; pairs past the head dim read pair 0 (in bounds, multiplied by a
    // zero query element, never written out).
    uint32_t pair_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pair_off[i] = d0 + 2 * i < hd ? (uint32_t)((d0 + 2 * i) * kElem) : 0u;
    // Odd head dims: the pair's second element, or its first again past the
    // head dim (in the row; its query element is zero).
    uint32_t pair_off2[ODD ? 4 : 1];
#pragma unroll
    for (int i = 0; i < (ODD ? 4 : 0); ++i)
      pair_off2[i] = d0 + 2 * i + 1 < hd ? pair_off[i] + kElem : pair_off[i];

    // Page-table window: lane i holds the physical id of unit page
    // win + dir * i (lanes past the unit's ends hold an end entry and are
    // never read). One load for all lanes, no branch.
    int win = pa;
    int tbl = 0;
    auto load_window = [&]() {
      const int e = win + dir * lane;
      tbl = table[min(max(e, 0), npg - 1)];
    };
    load_window();

    // Loader state: the page being loaded (lpa, its id) and the next step in
    // it; `loading` turns false when the unit or the tickets run out.
    int lpa = pa;
    int lsub = 0;
    int lpid = 0;
    bool loading = true;
    int next_ticket = 0;
    bool start_page = true;
    int cnt = 0;  // pages of this unit taken by this wave
    // Per ring slot: is it a real step, its first key position, page usable,
    // keys of the page from its first key on (KPS unless the page is ragged).
    bool s_real[NBUF];
    int s_t0[NBUF];
    bool s_ok[NBUF];
    int s_kin[NBUF];
    int64_t last_off = 0;
    int64_t last_soff = 0;  // 8-bit: scale element of the step's first key
    // Ragged pages: rows this lane's loads move back so that the last,
    // partial step of a page stays inside it (this lane's key, the keys of
    // its value pair); the keys they duplicate are masked.
    int last_dk = 0, last_dv0 = 0, last_dv1 = 0;

    f16x8 kb[NBUF][NV], vb[NBUF][NV];
    // 8-bit: this lane's key scale and the value scales of its pair's keys
    // (own, other), kept apart until the step is computed so that no
    // instruction waits on them at load time.
    f16 ksb[NBUF], vs_own_b[NBUF], vs_other_b[NBUF];

    auto load_step = [&](int u) {
      if (loading && start_page) {
        // Start page lpa: its ticket was granted (`pending`); take the ticket
        // of the page after it now, while this one loads.
        if (!pending) {
          loading = false;
        } else {
          pending = false;
          ++cnt;
          ++taken;
          const int idx = dir * (lpa - win);
          if (idx < 0 || idx >= kTablePages) {
            // Rare: the next 64 entries. Read here, so the common path never
            // waits on this load.
            win = lpa;
            load_window();
            lpid = __builtin_amdgcn_readlane(tbl, 0);
          } else {
            lpid = __builtin_amdgcn_readlane(tbl, idx);
          }
          start_page = false;
          next_ticket = take_ticket();
        }
      }
      if (loading) {
        const bool ok = lpid >= 0 && lpid < p.arena_pages;
        const int pid = ok ? lpid : 0;
        last_off = (int64_t)pid * p.page_bytes + lsub * KPS * p.row_bytes;
        if constexpr (Q8) last_soff = (int64_t)pid * p.scale_page + lsub * KPS * p.scale_row;
        s_real[u] = true;
        s_t0[u] = (first_page + lpa) * P + lsub * KPS;
        s_ok[u] = ok;
        s_kin[u] = KPS;
        if (p.ragged) {
          const int kin = min(KPS, P - lsub * KPS);
          s_kin[u] = kin;
          last_dk = min(lk, kin - 1) - lk;
          last_dv0 = min(2 * kp, kin - 1) - 2 * kp;
          last_dv1 = min(2 * kp + 1, kin - 1) - (2 * kp + 1);
        }
        if (++lsub == spp) {
          lsub = 0;
          start_page = true;
          lpa += dir;
          // The ticket taken for the next page decides whether it is ours;
          // past the unit's end it is the next unit's first page.
          pending = granted(next_ticket);
          if (lpa < 0 || lpa >= npg) loading = false;
        }
      } else {
        s_real[u] = false;
      }
      // Once the unit is done the ring keeps reloading the last step (never
      // used), so every slot always has one load in flight and the wait
      // counts stay those of a steady ring. Those reloads drop the lanes'
      // offsets: every lane of an instruction reads the same 16 bytes, one
      // cache line per instruction instead of a whole step (at one page per
      // wave, a 2-deep ring otherwise doubles the L2 reads, an 8-deep one
      // multiplies them by 8).
      // Every per-lane term goes: the lane's column and row offsets, the
      // ragged shifts (which move rows back by up to the lane's own row, so
      // without the row they would point before the page) and the second
      // key row of a pair. What stays is the step's first row (inside the
      // page) plus chunk offsets inside that row. (A 1-deep ring reloads
      // once per unit; it keeps the plain reload and its registers.)
      const bool dummy = NBUF > 1 && !s_real[u];
      const uint32_t lm = dummy ? 0u : ~0u;
      const int dk = dummy ? 0 : last_dk;                 // K row shift
      const int dv0 = dummy ? 0 : last_dv0;               // first value row of the pair
      const int dv1 = dummy ? 0 : 1 + last_dv1;           // second value row of the pair
      const int dvo = dummy ? 0 : (hi ? last_dv1 : last_dv0);  // this lane's value row shift
      const int dvx = dummy ? 0 : (hi ? last_dv0 : last_dv1);  // the other key's
      const int rb = p.row_bytes;
      const char* kq = kbase + last_off + (lane_off & lm) + dk * rb;
      const char* vq = vbase + last_off + (v_off & lm);
      if constexpr (GEN) {
        // Four element pairs of this lane's key row, K then V.
        const char* vk = vq + dk * rb;
        if constexpr (Q8 && ODD) {
          uint32_t kw[4], vw[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint8_t* k8 = reinterpret_cast<const uint8_t*>(kq);
            const uint8_t* v8 = reinterpret_cast<const uint8_t*>(vk);
            kw[i] = (uint32_t)k8[pair_off[i] & lm] | (uint32_t)k8[pair_off2[i] & lm] << 8;
            vw[i] = (uint32_t)v8[pair_off[i] & lm] | (uint32_t)v8[pair_off2[i] & lm] << 8;
          }
          kb[u][0] = __builtin_bit_cast(
              f16x8, i32x4{(int)(kw[0] | kw[1] << 16), (int)(kw[2] | kw[3] << 16), 0, 0});
          vb[u][0] = __builtin_bit_cast(
              f16x8, i32x4{(int)(vw[0] | vw[1] << 16), (int)(vw[2] | vw[3] << 16), 0, 0});
          const int so = dk * p.scale_row;
          ksb[u] = p.kscale[last_soff + (ks_off & lm) + so];
          vs_own_b[u] = p.vscale[last_soff + (vs_own & lm) + so];
        } else if constexpr (Q8) {
          uint32_t kw[4], vw[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kw[i] = *reinterpret_cast<const uint16_t*>(kq + (pair_off[i] & lm));
            vw[i] = *reinterpret_cast<const uint16_t*>(vk + (pair_off[i] & lm));
          }
          kb[u][0] = __builtin_bit_cast(
              f16x8, i32x4{(int)(kw[0] | kw[1] << 16), (int)(kw[2] | kw[3] << 16), 0, 0});
          vb[u][0] = __builtin_bit_cast(
              f16x8, i32x4{(int)(vw[0] | vw[1] << 16), (int)(vw[2] | vw[3] << 16), 0, 0});
          const int so = dk * p.scale_row;
          ksb[u] = p.kscale[last_soff + (ks_off & lm) + so];
          vs_own_b[u] = p.vscale[last_soff + (vs_own & lm) + so];
        } else if constexpr (ODD) {
          i32x4 kw, vw;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint16_t* k16a = reinterpret_cast<const uint16_t*>(kq + (pair_off[i] & lm));
            const uint16_t* k16b = reinterpret_cast<const uint16_t*>(kq + (pair_off2[i] & lm));
            const uint16_t* v16a = reinterpret_cast<const uint16_t*>(vk + (pair_off[i] & lm));
            const uint16_t* v16b = reinterpret_cast<const uint16_t*>(vk + (pair_off2[i] & lm));
            kw[i] = (int)((uint32_t)*k16a | (uint32_t)*k16b << 16);
            vw[i] = (int)((uint32_t)*v16a | (uint32_t)*v16b << 16);
          }
          kb[u][0] = __builtin_bit_cast(f16x8, kw);
          vb[u][0] = __builtin_bit_cast(f16x8, vw);
        } else {
          i32x4 kw, vw;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kw[i] = *reinterpret_cast<const int*>(kq + (pair_off[i] & lm));
            vw[i] = *reinterpret_cast<const int*>(vk + (pair_off[i] & lm));
          }
          kb[u][0] = __builtin_bit_cast(f16x8, kw);
          vb[u][0] = __builtin_bit_cast(f16x8, vw);
        }
      } else if constexpr (MF && Q8) {
        // 16 int8 elements (two chunks) of this lane's key per load, K and
        // V of the same key, and that key's two scales.
#pragma unroll
        for (int j = 0; j < NV / 2; ++j) {
          kb[u][j] = *reinterpret_cast<const f16x8*>(kq + 64 * j);
          vb[u][j] = *reinterpret_cast<const f16x8*>(vq + dk * rb + 64 * j);
        }
        const int so = dk * p.scale_row;
        ksb[u] = p.kscale[last_soff + (ks_off & lm) + so];
        vs_own_b[u] = p.vscale[last_soff + (vs_own & lm) + so];
      } else if constexpr (Q8) {
        kb[u][0] = *reinterpret_cast<const f16x8*>(kq);
        const uint2 va = *reinterpret_cast<const uint2*>(vq + dv0 * rb);
        const uint2 vc = *reinterpret_cast<const uint2*>(vq + dv1 * rb);
        vb[u][0] = __builtin_bit_cast(f16x8, i32x4{(int)va.x, (int)va.y, (int)vc.x, (int)vc.y});
        const f16* ks = p.kscale + last_soff;
        const f16* vs = p.vscale + last_soff;
        ksb[u] = ks[(ks_off & lm) + dk * p.scale_row];
        vs_own_b[u] = vs[(vs_own & lm) + dvo * p.scale_row];
        vs_other_b[u] = vs[(vs_other & lm) + dvx * p.scale_row];
      } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          kb[u][v] = *reinterpret_cast<const f16x8*>(kq + 2 * DC * v);
          vb[u][v] = *reinterpret_cast<const f16x8*>(
              PV2 ? vq + (v ? dv1 : dv0) * rb : vq + dk * rb + 2 * DC * v);
        }
      }
    };

    // 8-bit matrix-core step: chunk h of a 16-byte int8 K piece and of the V
    // piece, converted exactly to fp16 (K) and to fp16(int8 x scale) (V,
    // rounded as the reference's gather does, paged_kv.py:285-292).
    auto q8_chunk = [&](const f16x8& kpiece, const f16x8& vpiece, int h, f16x2 vsc, f16x8& kc,
                        f16x8& vc) {
      const i32x4 kr = __builtin_bit_cast(i32x4, kpiece);
      const i32x4 vr8 = __builtin_bit_cast(i32x4, vpiece);
      f16x2 kq2[4], vq2[4];
#pragma unroll
      for (int w2 = 0; w2 < 2; ++w2) {
        const uint32_t kf = (uint32_t)kr[2 * h + w2] ^ 0x80808080u;
        const uint32_t vf = (uint32_t)vr8[2 * h + w2] ^ 0x80808080u;
        kq2[2 * w2] = bytes_to_f16x2(kf, 0x04010400u);
        kq2[2 * w2 + 1] = bytes_to_f16x2(kf, 0x04030402u);
        vq2[2 * w2] = bytes_to_f16x2(vf, 0x04010400u) * vsc;
        vq2[2 * w2 + 1] = bytes_to_f16x2(vf, 0x04030402u) * vsc;
      }
      kc = f16x8{kq2[0][0], kq2[0][1], kq2[1][0], kq2[1][1],
                 kq2[2][0], kq2[2][1], kq2[3][0], kq2[3][1]};
      vc = f16x8{vq2[0][0], vq2[0][1], vq2[1][0], vq2[1][1],
                 vq2[2][0], vq2[2][1], vq2[3][0], vq2[3][1]};
    };

    // Matrix-core step after the S product: the scores (times their keys'
    // scales at 8 bits; lane k % 16 loaded the scale of key k), the masks of
    // a boundary step, the lazy running max, P^T, and O^T += V^T P^T through
    // this wave's LDS tile. With stores_v the step's V chunks `vc` go into
    // the tile here (masked keys' rows zeroed first); otherwise the caller
    // has stored them.
    auto mf_back = [&](const f32x4& sacc, int t0, int lim, float ks_own, f16x8(&vc)[NV],
                       auto stores_v) {
      // 8-bit: each score times its key's scale (metal_kernels.py:52
      // KEY_SCALE); lane k % 16 loaded the scale of key k.
      float ksc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
      if constexpr (Q8) {
#pragma unroll
        for (int e = 0; e < 4; ++e) ksc[e] = __shfl(ks_own, 4 * mg + e);
      }
      float sr[4], x[4];  // scores in log2 units, and minus the running max
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float raw = Q8 ? sacc[e] * ksc[e] : sacc[e];
        if (p.softcap > 0.0f) {
          const float ex = __builtin_amdgcn_exp2f(raw * p.cap_in);
          sr[e] = (1.0f - 2.0f * __builtin_amdgcn_rcpf(ex + 1.0f)) * p.cap_out;
        } else {
          sr[e] = raw * p.scale_log2;
        }
        x[e] = sr[e] - m[0];
      }
      if (!(t0 >= first && t0 + 16 <= lim)) {
        // Boundary step: scores of keys outside [first, lim) are masked,
        // and the V row this lane loaded is zeroed if its key is.
        bool any = false;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = t0 + 4 * mg + e;
          const bool ok = t >= first && t < lim;
          sr[e] = ok ? sr[e] : -INFINITY;
          x[e] = ok ? x[e] : -INFINITY;
          any |= ok;
        }
        if (!__any(any)) return;
        if constexpr (decltype(stores_v)::value) {
          const bool vok = t0 + lk >= first && t0 + lk < lim;
#pragma unroll
          for (int c = 0; c < NV; ++c) vc[c] = zero_unless(vc[c], vok);
        }
      }
      if (__any(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])) > kSlack)) {
        // Rare: raise each head's running max to its largest score of
        // the step (every head sees the step's visible keys, so the max
        // is finite) and rescale its sum and outputs.
        float hm = fmaxf(fmaxf(sr[0], sr[1]), fmaxf(sr[2], sr[3]));
        hm = fmaxf(hm, __shfl_xor(hm, 16));
        hm = fmaxf(hm, __shfl_xor(hm, 32));
        const float mn = fmaxf(m[0], hm);
        const float f = __builtin_amdgcn_exp2f(m[0] - mn);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = sr[e] - mn;
        m[0] = mn;
        l[0] *= f;
#pragma unroll
        for (int i = 0; i < D / 16; ++i) ob[i] *= f;
      }
      // P^T, the B operand of O^T += V^T P^T as the accumulator holds it;
      // the sum uses the same rounded probabilities.
      f16x4 pb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pr = __builtin_amdgcn_exp2f(x[e]);
        if constexpr (BFM) {
          const bf16 r16 = (bf16)pr;
          pb[e] = __builtin_bit_cast(f16, r16);
          l[0] += (float)r16;
        } else {
          pb[e] = (f16)pr;
          l[0] += (float)pb[e];
        }
      }
      // V^T through this wave's LDS tile: the row pieces as loaded, then
      // a transposed read gives lane l element 16 i + l % 16 of keys
      // 4 mg .. 4 mg + 3 (in-order LDS: the next step's stores follow
      // these reads).
      f16* const vt = s_vt + w * 16 * kVRow;
      if constexpr (decltype(stores_v)::value) {
#pragma unroll
        for (int c = 0; c < NV; ++c)
          *reinterpret_cast<f16x8*>(vt + lk * kVRow + mf_elem(c)) = vc[c];
      }
      const f16* const vr = vt + (4 * mg + ((lane & 15) >> 2)) * kVRow + 4 * (lane & 3);
#pragma unroll
      for (int i = 0; i < D / 16; ++i) ob[i] = mfma_k16<BFM>(read_tr(vr + 16 * i), pb, ob[i]);
    };

    // 8-bit matrix-core step with one step in flight (D >= 256), first part:
    // the step's V chunks converted (8-bit) and stored into the LDS tile,
    // masked keys' rows zeroed, and S^T = K Q^T. It consumes every register
    // the step's loads filled, so the next step's loads can be issued before
    // the softmax and p.v (mf_back) instead of after them.
    auto mf_front = [&](int u, f32x4& sacc, int& t0, int& lim, float& ks_own) -> bool {
      if (!s_ok[u]) return false;  // released or out-of-range page: masked
      t0 = s_t0[u];
      lim = min(len, t0 + s_kin[u]);
      const bool vok = (t0 >= first && t0 + 16 <= lim) || (t0 + lk >= first && t0 + lk < lim);
      f16* const vt = s_vt + w * 16 * kVRow;
      sacc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      ks_own = 1.0f;
      if constexpr (Q8) {
        ks_own = (float)ksb[u] * qscale;
        const f16x2 vsc = {vs_own_b[u], vs_own_b[u]};
#pragma unroll
        for (int j = 0; j < NV / 2; ++j) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            f16x8 kc, vc;
            q8_chunk(kb[u][j], vb[u][j], h, vsc, kc, vc);
            *reinterpret_cast<f16x8*>(vt + lk * kVRow + mf_elem(2 * j + h)) =
                zero_unless(vc, vok);
            sacc = mfma_k32<BFM>(kc, qb[2 * j + h], sacc);
          }
        }
      }
      return true;
    };

    auto compute_step = [&](int u) {
      if (!s_ok[u]) return;  // released or out-of-range page: masked
      const int t0 = s_t0[u];
      f16x8(&kd)[NV] = kb[u];
      f16x8(&vd)[NV] = vb[u];
      if constexpr (MF) {
        // 8-bit: K and V chunks converted exactly to fp16 (int8 pieces of
        // two chunks per load); V rows times their scale, rounded to fp16
        // as the reference's gather does (paged_kv.py:285-292).
        f16x8 kc[NV], vc[NV];
        if constexpr (Q8) {
          const f16x2 vsc = {vs_own_b[u], vs_own_b[u]};
#pragma unroll
          for (int j = 0; j < NV / 2; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) q8_chunk(kd[j], vd[j], h, vsc, kc[2 * j + h], vc[2 * j + h]);
        } else {
#pragma unroll
          for (int c = 0; c < NV; ++c) {
            kc[c] = kd[c];
            vc[c] = vd[c];
          }
        }
        // S^T = K Q^T over the step's 16 keys on the matrix cores: this
        // lane holds keys 4 mg .. 4 mg + 3 of head lane % 16.
        f32x4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NV; ++c) sacc = mfma_k32<BFM>(kc[c], qb[c], sacc);
        mf_back(sacc, t0, min(len, t0 + s_kin[u]), Q8 ? (float)ksb[u] * qscale : 1.0f, vc,
                std::true_type{});
        return;
      } else {
      // q.k for every head of the group: v_dot2 over this lane's slice,
      // then the butterfly over the R lanes of the key.
      // This lane's key elements as fp16 pairs (8-bit: converted exactly).
      f16x2 kp2[EPL / 2];
      if constexpr (Q8) {
        const i32x4 raw = __builtin_bit_cast(i32x4, kd[0]);
#pragma unroll
        for (int j = 0; j < EPL / 4; ++j) {
          const uint32_t flipped = (uint32_t)raw[j] ^ 0x80808080u;
          kp2[2 * j] = bytes_to_f16x2(flipped, 0x04010400u);
          kp2[2 * j + 1] = bytes_to_f16x2(flipped, 0x04030402u);
        }
      } else {
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
          for (int i = 0; i < 4; ++i) kp2[4 * v + i] = f16x2{kd[v][2 * i], kd[v][2 * i + 1]};
      }
      float s[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc;
        if constexpr (BFM) {
          acc = dot2_first_bf16(__builtin_bit_cast(bf16x2, q[g][0]),
                                __builtin_bit_cast(bf16x2, kp2[0]));
#pragma unroll
          for (int i = 1; i < EPL / 2; ++i)
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q[g][i]),
                                                  __builtin_bit_cast(bf16x2, kp2[i]), acc, false);
        } else {
          acc = dot2_first(q[g][0], kp2[0]);
#pragma unroll
          for (int i = 1; i < EPL / 2; ++i) acc = __builtin_amdgcn_fdot2(q[g][i], kp2[i], acc, false);
        }
        s[g] = acc;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) s[g] = group_sum<R>(s[g]);
      // Scores in log2 units per unit of s (8-bit: times this key's scale,
      // metal_kernels.py:52 KEY_SCALE).
      float sl2 = p.scale_log2;
      if constexpr (Q8) {
        const float ksf = (float)ksb[u] * qscale;
        sl2 *= ksf;
        if (p.softcap > 0.0f) {
#pragma unroll
          for (int g = 0; g < G; ++g) s[g] *= ksf;
        }
      }
      // x = score - running max, in log2 units; softcap c * tanh(x / c)
      // (metal_kernels.py:53) as c * (1 - 2 / (e^(2x/c) + 1)).
      float x[G];
      if (p.softcap > 0.0f) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float e = __builtin_amdgcn_exp2f(s[g] * p.cap_in);
          x[g] = (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f)) * p.cap_out - m[g];
        }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) x[g] = __builtin_fmaf(s[g], sl2, -m[g]);
      }
      // Keys of the step past its page (ragged pages) are masked like keys
      // past the length.
      const int lim = min(len, t0 + s_kin[u]);
      if (!(t0 >= first && t0 + KPS <= lim)) {
        // Boundary step. A step with no visible key is skipped: before the
        // first visible key the running max is still -inf, and -inf - -inf
        // would poison the sums. Rows outside [first, len) may hold
        // anything, so their scores are masked and their values zeroed.
        const int t = t0 + kk;
        const bool valid = t >= first && t < lim;
        if (!__any(valid)) return;
#pragma unroll
        for (int g = 0; g < G; ++g) x[g] = valid ? x[g] : -INFINITY;
        if constexpr (GEN) {
          vd[0] = zero_unless(vd[0], valid);
          if constexpr (Q8) vs_own_b[u] = valid ? vs_own_b[u] : (f16)0.0f;
        } else if constexpr (Q8) {
          // Zero bytes are zero values; the scales of masked keys may hold
          // anything, so they are zeroed too.
          const int ta = t0 + 2 * kp;
          const bool v0 = ta >= first && ta < lim, v1 = ta + 1 >= first && ta + 1 < lim;
          i32x4 bits = __builtin_bit_cast(i32x4, vd[0]);
          bits.x = v0 ? bits.x : 0;
          bits.y = v0 ? bits.y : 0;
          bits.z = v1 ? bits.z : 0;
          bits.w = v1 ? bits.w : 0;
          vd[0] = __builtin_bit_cast(f16x8, bits);
          const bool own_ok = hi ? v1 : v0, other_ok = hi ? v0 : v1;
          vs_own_b[u] = own_ok ? vs_own_b[u] : (f16)0.0f;
          vs_other_b[u] = other_ok ? vs_other_b[u] : (f16)0.0f;
        } else if constexpr (PV2) {
          const int ta = t0 + 2 * kp;
#pragma unroll
          for (int v = 0; v < NV; ++v) vd[v] = zero_unless(vd[v], ta + v >= first && ta + v < lim);
        } else {
#pragma unroll
          for (int v = 0; v < NV; ++v) vd[v] = zero_unless(vd[v], valid);
        }
      }
      bool grow = false;
#pragma unroll
      for (int g = 0; g < G; ++g) grow |= x[g] > kSlack;
      if (__any(grow)) {
        // Rare: a score passed the running max by 2^8 (always so for the
        // first visible key, while the max is -inf). Raise the max to the
        // wave's largest score and rescale what was summed so far. The
        // scores are recomputed from s: x + m would be inf - inf there.
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float sc;
          if (p.softcap > 0.0f) {
            const float e = __builtin_amdgcn_exp2f(s[g] * p.cap_in);
            sc = (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f)) * p.cap_out;
          } else {
            sc = s[g] * sl2;
          }
          sc = x[g] == -INFINITY ? -INFINITY : sc;  // masked keys stay out
          const float mn = fmaxf(m[g], wave_max(sc));
          const float f = __builtin_amdgcn_exp2f(m[g] - mn);
          x[g] = sc - mn;
          m[g] = mn;
          l[g] *= f;
#pragma unroll
          for (int i = 0; i < OPL; ++i) o[g][i] *= f;
        }
      }
      if constexpr (PV2) {
        // V element pairs (this lane's key, the other key of its pair),
        // shared by all heads.
        f16x2 vv[8];
        if constexpr (Q8) {
          // Bytes of keys 2 kp (dwords x, y) and 2 kp + 1 (z, w), elements
          // r2 * 8 .. r2 * 8 + 7: interleave them (this lane's key first),
          // convert exactly, then weight by the keys' value scales
          // (metal_kernels.py:58 VALUE_SCALE).
          const i32x4 raw = __builtin_bit_cast(i32x4, vd[0]);
          const f16x2 vsp = f16x2{vs_own_b[u], vs_other_b[u]};
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const uint32_t a = (uint32_t)raw[j] ^ 0x80808080u;
            const uint32_t c = (uint32_t)raw[2 + j] ^ 0x80808080u;
            const uint32_t lo = __builtin_amdgcn_perm(a, c, sel8_lo);  // elements 4j, 4j + 1
            const uint32_t hi2 = __builtin_amdgcn_perm(a, c, sel8_hi); // elements 4j + 2, 4j + 3
            vv[4 * j] = bytes_to_f16x2(lo, 0x04010400u) * vsp;
            vv[4 * j + 1] = bytes_to_f16x2(lo, 0x04030402u) * vsp;
            vv[4 * j + 2] = bytes_to_f16x2(hi2, 0x04010400u) * vsp;
            vv[4 * j + 3] = bytes_to_f16x2(hi2, 0x04030402u) * vsp;
          }
        } else {
          const i32x4 va = __builtin_bit_cast(i32x4, vd[0]);  // key 2 kp
          const i32x4 vb = __builtin_bit_cast(i32x4, vd[1]);  // key 2 kp + 1
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            vv[2 * j] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(va[j], vb[j], sel_lo));
            vv[2 * j + 1] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(va[j], vb[j], sel_hi));
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          // Probabilities of the pair's two keys as fp16: this lane holds its
          // own key's, lane ^ R the other's. The sum uses the same rounded
          // values, so the weights stay a normalised combination.
          const float pr = __builtin_amdgcn_exp2f(x[g]);
          const float other = pair_swap<R>(pr);
          if constexpr (BFM) {
            const bf16x2 pp = bf16x2{(bf16)pr, (bf16)other};
            l[g] = __builtin_amdgcn_fdot2_f32_bf16(pp, bf16x2{(bf16)1.0f, (bf16)1.0f}, l[g], false);
#pragma unroll
            for (int i = 0; i < 8; ++i)
              o[g][i] = __builtin_amdgcn_fdot2_f32_bf16(pp, __builtin_bit_cast(bf16x2, vv[i]),
                                                        o[g][i], false);
          } else {
            const f16x2 pp = f16x2{(f16)pr, (f16)other};
            l[g] = __builtin_amdgcn_fdot2(pp, f16x2{(f16)1.0f, (f16)1.0f}, l[g], false);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[g][i] = __builtin_amdgcn_fdot2(pp, vv[i], o[g][i], false);
          }
        }
      } else if constexpr (Q8) {
        // Generic 8-bit: this lane's key's eight value bytes, weighted by the
        // probability times the key's value scale (metal_kernels.py:58).
        const i32x4 raw = __builtin_bit_cast(i32x4, vd[0]);
        float vf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          vf[i] = (float)(int)__builtin_amdgcn_sbfe(raw[i / 4], 8 * (i % 4), 8);
        const float vsf = (float)vs_own_b[u];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pr = __builtin_amdgcn_exp2f(x[g]);
          l[g] += pr;
          const float wv = pr * vsf;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[g][i] = __builtin_fmaf(wv, vf[i], o[g][i]);
        }
      } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pr = __builtin_amdgcn_exp2f(x[g]);
          l[g] += pr;
#pragma unroll
          for (int v = 0; v < NV; ++v) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
              o[g][8 * v + i] = __builtin_fmaf(
                  pr, BFM ? (float)__builtin_bit_cast(bf16x8, vd[v])[i] : (float)vd[v][i],
                  o[g][8 * v + i]);
          }
        }
      }
      }  // not MF
    };

#pragma unroll
    for (int u = 0; u < NBUF; ++u) load_step(u);
    if constexpr (MF && Q8 && NBUF == 1) {
      // One step in flight (8-bit, D >= 256): wait for it, consume its
      // registers (mf_front), issue the next step's loads, then finish the
      // step (mf_back) while they are in flight. On the Gemma 4 global
      // layer at 8 bits, 152 -> 135 us; the 16-bit kernels, whose steps are
      // twice the bytes, were 1-3% slower this way and keep the plain ring.
      do {
        wait_vmem<0>();
        f32x4 sacc;
        int t0 = 0, lim = 0;
        float ks_own = 1.0f;
        const bool live = s_real[0] && mf_front(0, sacc, t0, lim, ks_own);
        load_step(0);
        if (live) mf_back(sacc, t0, lim, ks_own, vb[0], std::false_type{});
      } while (s_real[0]);
    } else {
      // The ring: every slot is waited for (its loads are complete once
      // only the other slots' remain), computed if it holds a real step and
      // reloaded, in issue order on every path, with the loop test at the
      // bottom; the compiler's wait counts then stay those of a steady ring.
      do {
#pragma unroll
        for (int u = 0; u < NBUF; ++u) {
          wait_vmem<(NBUF - 1) * Gm::LOADS>();
          if (s_real[u]) compute_step(u);
          load_step(u);
        }
      } while (s_real[0]);
    }
    // `pending` now tells whether the page after this unit is ours too.

    if constexpr (MF) {
      // Matrix-core kernels: O^T is complete in the accumulators (lane l
      // holds elements 16 i + 4 mg .. + 3 of head l % 16); the sum of each
      // head is spread over its four lanes l % 16 + 16 j.
      float lt = l[0];
      lt += __shfl_xor(lt, 16);
      lt += __shfl_xor(lt, 32);
      const int head = lane & 15;
      if (cnt == npg && !p.local) {
        if (head < hpu) {  // the whole unit: normalise and write
          const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
          f16* const dst = p.out + ((int64_t)b * p.hq + h0 + head) * D + 4 * mg;
#pragma unroll
          for (int i = 0; i < D / 16; ++i) {
            f16x4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (BF)
                y[e] = __builtin_bit_cast(f16, (bf16)(ob[i][e] * inv));
              else
                y[e] = (f16)(ob[i][e] * inv);
            }
            *reinterpret_cast<f16x4*>(dst + 16 * i) = y;
          }
        }
      } else if (head < hpu) {
        // Cut unit: the unnormalised partial, slot chosen as below.
        // (Local mode: this wave's LDS slot.)
        const bool holds_start = back ? !pending : first_unit;
        const int64_t slot = p.local ? w : 2 * vw + (holds_start ? 0 : 1);
        float* const dst = (p.local ? s_lo : p.part_o) + (slot * hpu + head) * D + 4 * mg;
#pragma unroll
        for (int i = 0; i < D / 16; ++i)
          *reinterpret_cast<float4*>(dst + 16 * i) =
              make_float4(ob[i][0], ob[i][1], ob[i][2], ob[i][3]);
        if (mg == 0) (p.local ? s_lml : p.part_ml)[slot * hpu + head] = make_float2(m[0], lt);
      }
    } else {
    // Fold the wave's key subsets (metal_kernels.py:63-81); every lane then
    // holds the totals of its elements. On the p.v pair path the lanes of
    // key pair kp write the heads g with g % NPAIR == kp, elements r2 * 8 ..;
    // otherwise the lanes of key subset kk write the heads g with
    // g % KPS == kk, in chunks.
    constexpr int kWriters = PV2 ? Gm::NPAIR : KPS;
    const int writer = PV2 ? kp : kk;
    const bool writes = PV2 || active;
    const int e0 = PV2 ? r2 * 8 : d0;      // first output element of this lane
    const int estride = PV2 ? 8 : DC;     // between its chunks of 8
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (PV2) {
        l[g] = pair_sum<R>(l[g]);
#pragma unroll
        for (int i = 0; i < OPL; ++i) o[g][i] = pair_sum<R>(o[g][i]);
      } else {
        l[g] = subset_sum<R>(l[g]);
#pragma unroll
        for (int i = 0; i < OPL; ++i) o[g][i] = subset_sum<R>(o[g][i]);
      }
    }
    if (cnt == npg && !p.local) {
      // The whole unit is here: normalise and write (metal_kernels.py:87-91).
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (g % kWriters != writer || !writes) continue;
        const float inv = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
        if constexpr (ODD) {
          // Elements below the real head dim, 2-byte stores.
          f16* dst = p.out + ((int64_t)b * p.hq + h0 + g) * hd;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (e0 + i >= hd) continue;
            const float y = o[g][i] * inv;
            if constexpr (BF)
              dst[e0 + i] = __builtin_bit_cast(f16, (bf16)y);
            else
              dst[e0 + i] = (f16)y;
          }
          continue;
        } else if constexpr (GEN) {
          // Element pairs below the real head dim, 4-byte stores.
          f16* dst = p.out + ((int64_t)b * p.hq + h0 + g) * hd;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (e0 + 2 * i >= hd) continue;
            const float y0 = o[g][2 * i] * inv, y1 = o[g][2 * i + 1] * inv;
            if constexpr (BF)
              *reinterpret_cast<bf16x2*>(dst + e0 + 2 * i) = bf16x2{(bf16)y0, (bf16)y1};
            else
              *reinterpret_cast<f16x2*>(dst + e0 + 2 * i) = f16x2{(f16)y0, (f16)y1};
          }
          continue;
        }
        f16* dst = p.out + ((int64_t)b * p.hq + h0 + g) * D + e0;
#pragma unroll
        for (int v = 0; v < OPL / 8; ++v) {
          if constexpr (BF) {
            bf16x8 y;
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = (bf16)(o[g][8 * v + i] * inv);
            *reinterpret_cast<bf16x8*>(dst + estride * v) = y;
          } else {
            f16x8 y;
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = (f16)(o[g][8 * v + i] * inv);
            *reinterpret_cast<f16x8*>(dst + estride * v) = y;
          }
        }
      }
    } else {
      // Cut unit: unnormalised partial (metal_kernels.py:93-101) in slot 0 if
      // the unit holds the first page of this wave's final range (the first
      // wave's first unit, the second wave's last), else in slot 1.
      // (Local mode: this wave's LDS slot.)
      const bool holds_start = back ? !pending : first_unit;
      const int64_t slot = p.local ? w : 2 * vw + (holds_start ? 0 : 1);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (g % kWriters != writer || !writes) continue;
        float* dst = (p.local ? s_lo : p.part_o) + (slot * G + g) * D + e0;
#pragma unroll
        for (int i = 0; i < OPL; i += 4)
          *reinterpret_cast<float4*>(dst + estride * (i / 8) + i % 8) =
              make_float4(o[g][i], o[g][i + 1], o[g][i + 2], o[g][i + 3]);
        if ((PV2 ? r2 : r) == 0)
          (p.local ? s_lml : p.part_ml)[slot * G + g] = make_float2(m[g], l[g]);
      }
    }
    }  // not MF
    first_unit = false;
    if (!pending) break;

    // The next unit along the wave's way (empty sequences hold no pages).
    if (!back) {
      if (++kvg == nkvg) {
        kvg = 0;
        do {
          ++b;
        } while (b < B && s_prefix[b + 1] == s_prefix[b]);
      }
      if (b >= B) break;  // cannot happen: tickets never pass the range
      npg = s_prefix[b + 1] - s_prefix[b];
      pa = 0;
    } else {
      if (--kvg < 0) {
        kvg = nkvg - 1;
        do {
          --b;
        } while (b >= 0 && s_prefix[b + 1] == s_prefix[b]);
      }
      if (b < 0) break;  // cannot happen: tickets never pass the range
      npg = s_prefix[b + 1] - s_prefix[b];
      pa = npg - 1;
    }
  }
  if (!p.local) {
    // The first wave of the pair records the meeting point for the merge.
    // (Fixed split: the merge knows the point without it.)
    if (!back && lane == 0 && !p.fixed) p.meet[pair] = taken;
    return;
  }
  // Local mode: the workgroup's unit from its waves' pieces, the same
  // log-sum-exp merge as the merge kernel (metal_kernels.py:103-124), waves
  // folded in a fixed order.
  __syncthreads();
  const int ub = lx / nkvg;
  const int ukvg = lx - ub * nkvg;
  const int ukvh = ukvg / p.nhg;
  const int uh0 = ukvh * p.gtot + (ukvg - ukvh * p.nhg) * hpu_k;
  for (int i = tid; i < hpu_k * D; i += kThreads) {
    const int head = i / D;
    const int d = i - head * D;
    if (d >= hd) continue;
    float top = -INFINITY;
    for (int x = 0; x < kWaves; ++x) top = fmaxf(top, s_lml[x * hpu_k + head].x);
    float sum = 0.0f, acc = 0.0f;
    if (top != -INFINITY) {
      for (int x = 0; x < kWaves; ++x) {
        const float2 ml = s_lml[x * hpu_k + head];
        if (ml.x == -INFINITY) continue;
        const float wt = __builtin_amdgcn_exp2f(ml.x - top);
        sum = __builtin_fmaf(wt, ml.y, sum);
        acc = __builtin_fmaf(wt, s_lo[(x * hpu_k + head) * D + d], acc);
      }
    }
    const float y = sum > 0.0f ? acc / sum : 0.0f;
    f16* const dst = p.out + ((int64_t)ub * p.hq + uh0 + head) * hd + d;
    if constexpr (BF)
      *dst = __builtin_bit_cast(f16, (bf16)y);
    else
      *dst = (f16)y;
  }
}

// Pass one (metal_kernels.py:18-101): the split kernel of every even head
// dim, template arguments as split_body's.
template <int D, int G, bool Q8, bool BF, bool GEN, bool MF>
__global__ __launch_bounds__(64 * split_waves(D, MF))
__attribute__((amdgpu_waves_per_eu(split_waves(D, MF) / 4)))
void paged_decode_kernel(const Params p) {
  split_body<D, G, Q8, BF, GEN, MF, false>(p);
}

// Pass one at an odd head dim (the reference's IN_HEAD guard takes any,
// metal_kernels.py:28-30): the generic kernel of padded width D with
// element-wise loads and stores, one query head per unit (a rare shape: its
// GQA groups read K/V once per head).
template <int D, bool Q8, bool BF>
__global__ __launch_bounds__(64 * split_waves(D, false))
__attribute__((amdgpu_waves_per_eu(split_waves(D, false) / 4)))
void paged_decode_odd_kernel(const Params p) {
  split_body<D, 1, Q8, BF, true, false, true>(p);
}

// The pieces of one unit for the merge kernels. The unit's pages [s, e) of
// the stream lie in the ranges of pairs qa..qb; pair q split its range
// [X, Xn) at M = X + meet[q] into the first wave's [X, M) and the second
// wave's [M, Xn). Each of these ranges that meets [s, e) holds one piece of
// the unit, in slot 0 of that wave if the range starts inside the unit, else
// in slot 1. Candidate pieces are numbered 2 (q - qa) + (second wave).
struct UnitPieces {
  int64_t s = 0, e = 0, total = 0;
  int pairs = 0, qa = 0, cand = 0;

  // Slot of candidate j, or -1 when that wave's range misses the unit.
  __device__ __forceinline__ int slot(const Params& p, int j) const {
    const int q = qa + (j >> 1);
    const int64_t X = range_start(q, total, pairs);
    const int64_t Xn = range_start(q + 1, total, pairs);
    // Fixed split: the first wave took the first half (no load, so the
    // merge saves a dependent trip).
    const int64_t M = X + (p.fixed ? fixed_front(Xn - X, p) : p.meet[q]);
    if ((j & 1) == 0)
      return X < M && X < e && M > s ? 2 * (2 * q) + (X >= s ? 0 : 1) : -1;
    return M < Xn && M < e && Xn > s ? 2 * (2 * q + 1) + (M >= s ? 0 : 1) : -1;
  }
};

// The pieces of unit kvg of sequence b; false when the split kernel already
// wrote the output (no visible page: zeros; one piece: that wave's result).
__device__ __forceinline__ bool unit_pieces(const Params& p, int b, int kvg, int lane,
                                            UnitPieces& u) {
  const int nkvg = p.hkv * p.nhg;
  const int pb0 = p.prefix[b];
  const int npg = p.prefix[b + 1] - pb0;
  if (npg == 0) return false;
  u.total = (int64_t)p.prefix[p.batch] * nkvg;
  u.pairs = stream_pairs(u.total, p);
  u.s = (int64_t)pb0 * nkvg + (int64_t)kvg * npg;
  u.e = u.s + npg;
  u.qa = pair_of(u.s, u.total, u.pairs);
  u.cand = 2 * (pair_of(u.e - 1, u.total, u.pairs) - u.qa + 1);
  if (u.cand == 2) {
    // Inside one pair's range: a single piece means one wave held the whole
    // unit and wrote it.
    const int sl = lane < 2 ? u.slot(p, lane) : -1;
    if (__popcll(__ballot(sl >= 0)) <= 1) return false;
  }
  return true;
}

// Merge kernel (metal_kernels.py:103-124): one workgroup of MW waves per
// (sequence, kv head group, head of the group) combines the unit's pieces
// (UnitPieces). Wave w takes the batches of kBatch candidates w, w + MW,
// ...: one lane per candidate reads its pair's meeting point, then the
// loads of all pieces of the batch go out together and the batch is
// combined at once against its own maximum with log-sum-exp weights (pieces
// whose max is -inf hold no visible key and weigh 0; a zero total gives 0,
// :116,122). Batches and waves are folded in a fixed order, so the result
// does not depend on timing.
template <int D, int G, bool BF, bool GEN>
__global__ __launch_bounds__(kMergeMaxWaves * 64) void paged_decode_merge_kernel(const Params p) {
  constexpr int kChunks = (D + 63) / 64;  // elements l, l + 64, ... of lane l
  constexpr int kBatch = 32 / kChunks;    // candidates whose loads go out together
  __shared__ float s_top[kMergeMaxWaves], s_sum[kMergeMaxWaves];
  __shared__ float s_acc[kMergeMaxWaves][kChunks * 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int mw = blockDim.x >> 6;
  const int uh = p.unit_heads;  // query heads of a unit (G slots, fewer used by MF)
  const int kvg = blockIdx.x / uh;
  const int g = blockIdx.x - kvg * uh;
  const int b = blockIdx.y;
  const int kvh = kvg / p.nhg;
  const int h = kvh * p.gtot + (kvg - kvh * p.nhg) * uh + g;
  const int hd = GEN ? p.head_dim : D;  // output row length (partials are D apart)
  f16* const dst = p.out + ((int64_t)b * p.hq + h) * hd;
  UnitPieces up;
  if (!unit_pieces(p, b, kvg, lane, up)) return;
  const int cand = up.cand;

  float top = -INFINITY, sum = 0.0f, acc[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) acc[c] = 0.0f;
  for (int base = w * kBatch; base < cand; base += mw * kBatch) {
    const int mine = lane < kBatch && base + lane < cand ? up.slot(p, base + lane) : -1;
    int sl[kBatch];
    float2 ml[kBatch];
    float part[kBatch][kChunks];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      sl[u] = __builtin_amdgcn_readlane(mine, u);
      const int64_t at = sl[u] < 0 ? 0 : sl[u];
      ml[u] = p.part_ml[at * uh + g];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        const int d = c * 64 + lane;
        part[u][c] = d < D ? p.part_o[(at * uh + g) * D + d] : 0.0f;
      }
    }
    float bt = -INFINITY;
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (sl[u] >= 0) bt = fmaxf(bt, ml[u].x);
    if (bt == -INFINITY) continue;  // no visible key in this batch
    float bs = 0.0f, ba[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) ba[c] = 0.0f;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float wt = sl[u] >= 0 ? __builtin_amdgcn_exp2f(ml[u].x - bt) : 0.0f;
      bs = __builtin_fmaf(wt, ml[u].y, bs);
#pragma unroll
      for (int c = 0; c < kChunks; ++c) ba[c] = __builtin_fmaf(wt, part[u][c], ba[c]);
    }
    lse_add<kChunks>(top, sum, acc, make_float2(bt, bs), ba);
  }
  if (mw > 1) {
    // Combine the waves: each publishes its maximum, rescales to the common
    // one and leaves its sums in LDS; wave 0 adds them in a fixed order.
    if (lane == 0) s_top[w] = top;
    __syncthreads();
    float all = -INFINITY;
    for (int x = 0; x < mw; ++x) all = fmaxf(all, s_top[x]);
    const float f = top == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(top - all);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) s_acc[w][c * 64 + lane] = acc[c] * f;
    if (lane == 0) s_sum[w] = sum * f;
    __syncthreads();
    if (w != 0) return;
    sum = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) acc[c] = 0.0f;
    for (int x = 0; x < mw; ++x) {
      sum += s_sum[x];
#pragma unroll
      for (int c = 0; c < kChunks; ++c) acc[c] += s_acc[x][c * 64 + lane];
    }
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
  for (int c = 0; c < kChunks; ++c)
    if (c * 64 + lane < hd) {
      if constexpr (BF)
        dst[c * 64 + lane] = __builtin_bit_cast(f16, (bf16)(acc[c] * inv));
      else
        dst[c * 64 + lane] = (f16)(acc[c] * inv);
    }
}

// Row-sliced merge: the same combination, with the workgroups of one head
// each taking one 64-element slice of its row (blockIdx.x = head x slices +
// slice), for calls with few heads and many pieces each (a few long
// sequences), where one workgroup per head would leave most CUs idle and
// read whole rows on the few it has. A wave's round takes kRound
// candidates: lane j reads candidate j's meeting point and (max, sum); the
// pieces' slices are read with 16-byte loads, four pieces per load (lanes
// 16 i .. 16 i + 15 read piece 4 k + i in load k). The round is weighted
// against its own maximum; the four lane groups are summed after the last
// round and the waves folded in a fixed order, as in the kernel above.
template <int D, int G, bool BF, bool GEN>
__global__ __launch_bounds__(kMergeMaxWaves * 64) void paged_decode_merge_sliced_kernel(
    const Params p) {
  constexpr int kSlices = (D + 63) / 64;
  constexpr int kLoads = kMergeSlicedRound / 4;  // 16-byte loads per lane in a round
  static_assert(kMergeSlicedRound <= 64 && D % 4 == 0, "one candidate per lane, float4 rows");
  __shared__ float s_top[kMergeMaxWaves], s_sum[kMergeMaxWaves];
  __shared__ float4 s_acc[kMergeMaxWaves][16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int mw = blockDim.x >> 6;
  const int uh = p.unit_heads;
  const int x = blockIdx.x / kSlices;
  const int kvg = x / uh;
  const int g = x - kvg * uh;
  const int b = blockIdx.y;
  const int kvh = kvg / p.nhg;
  const int h = kvh * p.gtot + (kvg - kvh * p.nhg) * uh + g;
  const int hd = GEN ? p.head_dim : D;
  const int e0 = 64 * (blockIdx.x - x * kSlices) + 4 * (lane & 15);  // this lane's 4 elements
  const int grp = lane >> 4;
  UnitPieces up;
  if (!unit_pieces(p, b, kvg, lane, up)) return;
  const int cand = up.cand;

  float top = -INFINITY, sum = 0.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int base = w * kMergeSlicedRound; base < cand; base += mw * kMergeSlicedRound) {
    const int sl = lane < kMergeSlicedRound && base + lane < cand ? up.slot(p, base + lane) : -1;
    const float2 ml = sl >= 0 ? p.part_ml[(int64_t)sl * uh + g] : make_float2(-INFINITY, 0.0f);
    float4 part[kLoads];
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const int at = __shfl(sl, 4 * k + grp);
      part[k] = at >= 0 && e0 < D
                    ? *reinterpret_cast<const float4*>(p.part_o + ((int64_t)at * uh + g) * D + e0)
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const float bt = wave_max(ml.x);
    if (bt == -INFINITY) continue;  // no visible key in this round
    const float wt = sl >= 0 ? __builtin_amdgcn_exp2f(ml.x - bt) : 0.0f;
    const float bs = group_sum<64>(wt * ml.y);
    float4 ba = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const float wk = __shfl(wt, 4 * k + grp);
      ba.x = __builtin_fmaf(wk, part[k].x, ba.x);
      ba.y = __builtin_fmaf(wk, part[k].y, ba.y);
      ba.z = __builtin_fmaf(wk, part[k].z, ba.z);
      ba.w = __builtin_fmaf(wk, part[k].w, ba.w);
    }
    const float mn = fmaxf(top, bt);
    const float fo = __builtin_amdgcn_exp2f(top - mn);  // 0 while top = -inf
    const float fn = __builtin_amdgcn_exp2f(bt - mn);
    top = mn;
    sum = sum * fo + bs * fn;
    acc.x = acc.x * fo + ba.x * fn;
    acc.y = acc.y * fo + ba.y * fn;
    acc.z = acc.z * fo + ba.z * fn;
    acc.w = acc.w * fo + ba.w * fn;
  }
  // The four lane groups hold the same elements of different pieces, all
  // against the wave's maximum.
  acc.x += __shfl_xor(acc.x, 16);
  acc.y += __shfl_xor(acc.y, 16);
  acc.z += __shfl_xor(acc.z, 16);
  acc.w += __shfl_xor(acc.w, 16);
  acc.x += __shfl_xor(acc.x, 32);
  acc.y += __shfl_xor(acc.y, 32);
  acc.z += __shfl_xor(acc.z, 32);
  acc.w += __shfl_xor(acc.w, 32);
  if (mw > 1) {
    if (lane == 0) s_top[w] = top;
    __syncthreads();
    float all = -INFINITY;
    for (int i = 0; i < mw; ++i) all = fmaxf(all, s_top[i]);
    const float f = top == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(top - all);
    if (lane < 16) s_acc[w][lane] = make_float4(acc.x * f, acc.y * f, acc.z * f, acc.w * f);
    if (lane == 0) s_sum[w] = sum * f;
    __syncthreads();
    if (w != 0) return;
    sum = 0.0f;
    acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int i = 0; i < mw; ++i) {
      sum += s_sum[i];
      const float4 a = s_acc[i][lane & 15];
      acc.x += a.x;
      acc.y += a.y;
      acc.z += a.z;
      acc.w += a.w;
    }
  }
  if (lane >= 16) return;
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  const float o[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
  f16* const dst = p.out + ((int64_t)b * p.hq + h) * hd;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (e0 + j < hd) {
      if constexpr (BF)
        dst[e0 + j] = __builtin_bit_cast(f16, (bf16)o[j]);
      else
        dst[e0 + j] = (f16)o[j];
    }
}

// ---------------------------------------------------------------------------
// Instantiations, one translation unit per element type.

using KernelFn = void (*)(Params);

struct KernelPair {
  KernelFn split = nullptr;
  KernelFn merge = nullptr;
  KernelFn merge_sliced = nullptr;  // one 64-element slice per workgroup
  int split_waves = kSplitWaves;    // waves of a split workgroup
  int ring = kNbuf;                 // K/V steps in flight per wave
  // The split kernel's template arguments <D, G, Q8, BF, GEN, MF> (the
  // merge kernels take <D, G, BF, GEN>), as instantiated; odd: the split
  // kernel is paged_decode_odd_kernel<D, Q8, BF> (G = 1, GEN).
  int d = 0, g = 0;
  bool q8 = false, bf = false, gen = false, mf = false, odd = false;
};

template <int D, int G, bool Q8, bool BF, bool GEN = false, bool MF = false>
KernelPair make_pair() {
  return {paged_decode_kernel<D, G, Q8, BF, GEN, MF>,
          paged_decode_merge_kernel<D, G, BF, GEN>,
          paged_decode_merge_sliced_kernel<D, G, BF, GEN>,
          split_waves(D, MF),
          ring_depth(D, G, Q8, GEN, MF),
          D, G, Q8, BF, GEN, MF};
}

// Odd head dims: one query head per unit, the generic merges.
template <int D, bool Q8, bool BF>
KernelPair make_odd_pair() {
  return {paged_decode_odd_kernel<D, Q8, BF>,
          paged_decode_merge_kernel<D, 1, BF, true>,
          paged_decode_merge_sliced_kernel<D, 1, BF, true>,
          split_waves(D, false),
          ring_depth(D, 1, Q8, true, false),
          D, 1, Q8, BF, true, false, true};
}

template <int D, bool Q8, bool BF, bool GEN = false>
KernelPair pair_for_g(int g) {
  switch (g) {
    case 1: return make_pair<D, 1, Q8, BF, GEN>();
    case 2: return make_pair<D, 2, Q8, BF, GEN>();
    case 3: return make_pair<D, 3, Q8, BF, GEN>();
    case 4: return make_pair<D, 4, Q8, BF, GEN>();
    case 5: return make_pair<D, 5, Q8, BF, GEN>();
    case 6: return make_pair<D, 6, Q8, BF, GEN>();
    case 7: return make_pair<D, 7, Q8, BF, GEN>();
    case 8: return make_pair<D, 8, Q8, BF, GEN>();
  }
  return {};
}

// Kernels of the head dims compiled for one element type (the fast paths):
// fp16 and bf16 64, 80, 96, 128, 256, 512; 8-bit 64, 128, 256, 512.
KernelPair kernels_f16(int d, int g);
KernelPair kernels_bf16(int d, int g);
KernelPair kernels_q8(int d, int g);
// 8-bit K/V with bf16 queries and output (bf16 models).
KernelPair kernels_q8_bf16(int d, int g);
// Generic kernels for any other even head dim up to 512, padded to `dp`, a
// power of two from 8 to 512.
KernelPair kernels_gen_f16(int dp, int g);
KernelPair kernels_gen_bf16(int dp, int g);
KernelPair kernels_gen_q8(int dp, int g);
KernelPair kernels_gen_q8_bf16(int dp, int g);
// Odd head dims, padded to `dp` (a power of two from 8 to 512), one query
// head per unit: fp16 and bf16 queries over 16-bit or 8-bit K/V.
KernelPair kernels_odd(int dp, bool q8, bool bf16);
// Matrix-core kernels (5 to 16 query heads per unit): head dims 64, 96,
// 128, 256 in fp16 and bf16; 64, 128, 256 over 8-bit K/V.
KernelPair kernels_mf(int d, bool bf16);
KernelPair kernels_mf_q8(int d);
KernelPair kernels_mf_q8_bf16(int d);
// Matrix-core kernels at D = 512 (fp16, bf16 and 8-bit): four-wave
// workgroups, accumulators in AGPRs; a translation unit built without the
// VGPR-only matrix-core form.
KernelPair kernels_mf512(bool q8, bool bf16);

}  // namespace pda_decode

#endif  // PDA_DECODE_H
