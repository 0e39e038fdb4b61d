// Paged prefill attention for MI355X (gfx950), C-ABI in pda.h
// (pda_paged_prefill_attention).
//
// Reference: PrefillBatch.attend (python/instinct/batches.py:84-132): a chunk
// of one sequence's prompt, tokens at positions [start, start + count), whose
// keys and values were written to the paged arena first; query p attends
// keys [first(p), p] (causal, aligned to the newest key; with a window W,
// first(p) = p - W + 1), the score is softcapped when asked
// (portable.py:173-188), and the output is [count, q_heads * head_dim]. The
// CUDA engine's counterpart is its prefill attention kernel
// (cuda/kernels.cu:260-304).
//
// MI355X design (a flash-attention tile loop on the matrix cores):
//  * Workgroup = 4 waves = one query head and 128 queries (32 per wave).
//    Keys are streamed in tiles of 64 (32 at D >= 256) through LDS, K and V
//    rows gathered from the pages of the sequence's table (either arena
//    layout). The LDS holds two tiles: the loads of tile t + 1 are issued
//    into registers before the math of tile t and stored to the other half
//    after it, one barrier per tile.
//  * D = 512: eight waves, two blocks of 32 queries; the four waves of a
//    block split the head dim (128 dims of Q and O each) and sum their
//    partial scores through LDS, so every wave of the block holds the same
//    scores and probabilities (see slices_for).
//  * Each wave computes S^T = K Q^T for its 32 queries with
//    v_mfma_f32_32x32x16_f16 (D / 16 instructions per key tile), Q held in
//    registers. In that product's accumulator a lane holds 16 keys of one
//    query; 8 of them per 16-key step are the B operand of the next product
//    O^T += V^T P^T (D / 32 x 2 instructions per tile), so the probabilities
//    never leave registers. The contraction pairs A and B by k-slot, so the
//    V^T operand takes the keys in the order the accumulator holds them:
//    two ds_read_b64_tr_b16 per operand give a lane four consecutive keys of
//    one dimension each.
//  * Online softmax per query in the log2 domain with a lazy running max
//    (rescale only when a score passes the max by 2^8), fp16 probabilities
//    into the matrix core, fp32 accumulation, normalised fp16 output. Masks
//    (causality, the window, unusable pages) are evaluated only on the tiles
//    that need them; a wave skips the math of tiles none of its queries see.
//  * Work order: the query tiles with the most keys start first, and the G
//    query heads that read one kv head's tile are dispatched back to back to
//    one XCD (workgroups go round robin over the 8 XCDs), so the L2 of that
//    XCD serves the tile to all of them.
//  * LDS rows are padded so that the 16 lanes of a 16-byte K read, and the
//    four rows of a transposed V read, fall on distinct banks.
//  * Other even head dims up to 512 (GEN) run the kernel of the next of
//    those widths: rows are gathered as element pairs (the row length is a
//    multiple of 4 bytes only), the pairs past the head dim are zero in Q, K
//    and V, and only the real dims are written. Odd head dims (ODD) do the
//    same one element at a time (paged_prefill_odd_kernel).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "pda.h"
#include "pda_internal.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kSlack = 8.0f;
constexpr int kWaves = 4;  // waves per workgroup (D <= 256)
// Waves that split the head dim: at D = 512 the query fragments and output
// accumulators of 32 queries do not fit one wave's registers, so four waves
// share 32 queries, each holding 128 dims of Q and O; a D = 512 workgroup has
// eight waves (two such query blocks). (Split the same way, D = 256 runs two
// waves per SIMD instead of one but was 2-5% slower: the score exchange
// costs more than the second wave hides.)
constexpr int slices_for(int d) { return d > 256 ? 4 : 1; }
constexpr int waves_for(int d) { return d > 256 ? 2 * kWaves : kWaves; }
// Queries per workgroup: 32 per query block.
constexpr int queries_for(int d) { return 32 * waves_for(d) / slices_for(d); }
constexpr int kXcds = 8;

struct PrefillParams {
  const f16* q;        // [count, hq, D]
  const void* k;       // arena: fp16, or int8 with per-(row, kv head) fp16 scales
  const void* v;
  const f16* kscale;   // 8-bit only: scale arenas
  const f16* vscale;
  int64_t scale_page;  // scale elements between pages,
  int32_t scale_head;  //   between kv heads of one page,
  int32_t scale_row;   //   between rows of one page and kv head
  const int32_t* table;
  const int32_t* images;  // [num_images, 2] image spans [begin, end) of positions
  int32_t num_images;
  f16* out;            // [count, hq, D]
  float* part_o;       // [splits, count, hq, D] unnormalised partial outputs (splits > 1)
  float2* part_ml;     // [splits, count, hq] (running max, sum) of each partial
  int64_t arena_pages;
  int64_t page_elems;  // elements between pages of the arena
  int32_t head_elems;  // between kv heads of one page
  int32_t row_elems;   // between rows of one page and kv head
  int32_t table_len;
  int32_t start;
  int32_t count;
  int32_t tiles;       // query tiles = ceil(count / queries per workgroup)
  int32_t splits;      // key ranges per (query tile, head)
  int32_t page_step;   // keys per tile / page_size when that divides, else 0
  int32_t hq;
  int32_t hkv;
  int32_t head_dim;    // row length of Q, K, V and the output (GEN: below D)
  int32_t page_size;
  int32_t window;
  float scale_log2;
  float softcap;
  float cap_in;   // 2 log2(e) scale / softcap
  float cap_out;  // softcap log2(e)
};

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ f16x4 read_tr(const f16* p) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p));
}

// One 32x32x16 matrix-core step on 16-bit operands held as fp16 bit patterns:
// fp16, or bf16 (BF) for bf16 models.
template <bool BF>
__device__ __forceinline__ f32x16 mfma16(const f16x8& a, const f16x8& b, const f32x16& c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// f32 -> the 16-bit element type (to nearest even), as an fp16 bit pattern.
template <bool BF>
__device__ __forceinline__ f16 round16(float x) {
  if constexpr (BF)
    return __builtin_bit_cast(f16, (bf16)x);
  else
    return (f16)x;
}

// Keys per tile: 64 (two 32-key blocks) where the registers allow it.
template <int D>
constexpr int blocks_per_tile() { return D <= 128 ? 2 : 1; }

// Q8: the arena holds int8 rows and fp16 scales; the gather dequantizes each
// row to fp16(int8 x scale) on its way into LDS, the values the reference's
// 8-bit gather hands to attention (paged_kv.py:285-292), and the rest of the
// kernel is the fp16 one.
// BF: queries, K/V and output in bf16 (bf16 models); every 16-bit value is
// moved as raw bits and only the matrix-core steps, the probabilities and the
// output rounding differ.
// GEN: head dim p.head_dim below D; D-wide tiles, zero past it.
// ODD (with GEN): an odd head dim; rows are 2-byte aligned (1-byte at 8
// bits), so the queries, the gather and the output move single elements.
template <int D, bool Q8, bool BF, bool GEN, bool ODD>
__device__ __forceinline__ void prefill_body(const PrefillParams p) {
  static_assert(!ODD || GEN, "odd head dims run the generic kernels");
  static_assert(!(Q8 && BF), "8-bit K/V dequantizes to fp16");
  constexpr int KB = blocks_per_tile<D>();  // 32-key blocks per tile
  constexpr int kKeys = 32 * KB;            // keys per tile
  constexpr int kSlices = slices_for(D);    // waves sharing one query block
  constexpr int kDW = D / kSlices;          // head dims per wave
  constexpr int kQ = queries_for(D);        // queries per workgroup
  constexpr int kW = waves_for(D);          // waves per workgroup
  constexpr int kT = 64 * kW;               // threads per workgroup
  // D = 512: one V tile in LDS (the partials take the second one's room); V
  // of tile t + 1 is stored at the top of iteration t + 1, after every wave
  // is done with V of tile t.
  constexpr bool kOneV = D > 256;
  constexpr int kGroups = 4 * KB;             // float4 groups of a lane's scores
  constexpr int kPer = kGroups / kSlices;     // groups each slice sums
  static_assert(kPer * kSlices == kGroups, "score groups per slice");
  constexpr int kKRow = D + 8;    // K row in LDS (halves): 16-lane 16-byte reads hit distinct banks
  // V row: the 4 rows of a transposed read hit distinct banks (a row is 16
  // banks past the previous one modulo 64).
  constexpr int kVRow = D % 64 == 32 ? D + 64 : D + 32;
  constexpr int kTpk = kT / kKeys;                     // gather threads per key
  constexpr int kPieces = D / 8 / kTpk;                // 16-byte pieces per thread and tile
  constexpr int kKeysPerWave = 64 / kTpk;              // keys one wave gathers
  static_assert(kPieces >= 1 && kPieces * kTpk * 8 == D, "tile shape");
  typedef typename std::conditional<kKeysPerWave == 16, uint16_t, uint8_t>::type okbits;
  typedef typename std::conditional<KB == 2, uint64_t, uint32_t>::type okword;
  static_assert(kKeysPerWave * kW == kKeys, "usable-key bits");
  __shared__ __align__(16) f16 s_k[2][kKeys * kKRow];
  __shared__ __align__(16) f16 s_v[kOneV ? 1 : 2][kKeys * kVRow];
  __shared__ __align__(8) okbits s_ok[2][kW];  // usable-key bits of the tile
  // D = 512: each wave's partial scores (over its dims), and the sums of
  // the query block's partials, kPer groups per wave.
  __shared__ __align__(16) float4 s_x[kSlices > 1 ? kW * kGroups : 1][64];
  __shared__ __align__(16) float4 s_y[kSlices > 1 ? kW * kPer : 1][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int n = lane & 31;   // query column of this lane
  const int hh = lane >> 5;  // which half of the key rows this lane holds
  const int qb = w / kSlices;       // this wave's 32-query block
  const int sl = w - qb * kSlices;  // and its head dims: [sl kDW, (sl + 1) kDW)

  // Work item. Logical order: query tiles from the last (most keys) to the
  // first, then key range, then kv head, then the G query heads of that kv
  // head. Workgroup ids go round robin over the XCDs; whole runs of G (the
  // workgroups reading the same K/V tiles) go to one XCD.
  const int G = p.hq / p.hkv;
  int item = blockIdx.x;
  const int runs = p.tiles * p.splits * p.hkv;
  const int full = runs / kXcds * kXcds;
  if (item < full * G) {
    const int x = item % kXcds, j = item / kXcds;
    item = ((j / G) * kXcds + x) * G + j % G;
  }
  const int run = item / G;
  const int h = (run % p.hkv) * G + (item - run * G);
  const int kvh = run % p.hkv;
  const int split = (run / p.hkv) % p.splits;
  const int tile = p.tiles - 1 - run / p.hkv / p.splits;

  const int q0 = tile * kQ;
  const int q1 = min(q0 + kQ, p.count);
  const int qi = q0 + 32 * qb + n;  // this lane's query (may be past count)
  const bool q_live = qi < p.count;
  const int qpos = p.start + qi;
  const int wq0 = q0 + 32 * qb;
  const bool wave_live = wq0 < p.count;
  const int wfirst = p.start + wq0;
  const int wlast = p.start + min(wq0 + 31, p.count - 1);

  // Query fragments (B operand of S^T = K Q^T): dims 16 c + 8 hh .. + 7 of
  // the wave's slice.
  f16x8 qf[kDW / 16];
  if constexpr (GEN) {
    // Element pairs, clamped into the row; zero past the head dim.
    const int hd = p.head_dim;
    const f16* qp = p.q + ((int64_t)(q_live ? qi : 0) * p.hq + h) * hd;
#pragma unroll
    for (int c = 0; c < kDW / 16; ++c) {
      i32x4 x;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = sl * kDW + 16 * c + 8 * hh + 2 * j;
        if constexpr (ODD) {
          const uint16_t* q16 = reinterpret_cast<const uint16_t*>(qp);
          const uint32_t lo = q16[min(d, hd - 1)], hi = q16[min(d + 1, hd - 1)];
          x[j] = (int)((q_live && d < hd ? lo : 0u) | (q_live && d + 1 < hd ? hi : 0u) << 16);
        } else {
          const int y = *reinterpret_cast<const int*>(qp + min(d, hd - 2));
          x[j] = q_live && d < hd ? y : 0;
        }
      }
      qf[c] = __builtin_bit_cast(f16x8, x);
    }
  } else {
    const f16* qp = p.q + ((int64_t)(q_live ? qi : 0) * p.hq + h) * D + sl * kDW + 8 * hh;
#pragma unroll
    for (int c = 0; c < kDW / 16; ++c) {
      const f16x8 x = *reinterpret_cast<const f16x8*>(qp + 16 * c);
      qf[c] = q_live ? x : f16x8{};
    }
  }

  f32x16 o[kDW / 32];
#pragma unroll
  for (int b = 0; b < kDW / 32; ++b) o[b] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  // Keys this workgroup needs: from the first visible key of its first query
  // (rounded down to a tile) to its last query.
  int last = p.start + q1 - 1;
  int kfirst = p.window > 0 ? max(0, p.start + q0 - p.window + 1) : 0;
  // Image spans (batches.py:107-118): a query inside one also sees the
  // span's later keys, whatever the window. The lane keeps its query's span
  // [img_lo, img_hi); the workgroup and each wave extend their key ranges to
  // the spans their queries touch (keys stop at the chunk's end).
  int img_lo = 0, img_hi = 0, wave_last = wlast;
  bool wave_img = false;
  for (int i = 0; i < p.num_images; ++i) {
    const int a = p.images[2 * i], b = min(p.images[2 * i + 1], p.start + p.count);
    if (a >= b) continue;
    if (qpos >= a && qpos < b) img_lo = a, img_hi = b;
    if (a <= last && b > p.start + q0) {
      last = max(last, b - 1);
      kfirst = min(kfirst, a);
    }
    if (wave_live && a <= wlast && b > wfirst) {
      wave_last = max(wave_last, b - 1);
      wave_img = true;
    }
  }
  const int kbase = kfirst / kKeys * kKeys;
  const int ntile = (last - kbase) / kKeys + 1;
  // This workgroup's key range: tiles [t_begin, t_end) of the ntile.
  const int t_begin = (int)((int64_t)ntile * split / p.splits);
  const int t_end = (int)((int64_t)ntile * (split + 1) / p.splits);

  // Gather: thread tid moves key tid / kTpk of a tile, 16-byte pieces
  // tid % kTpk + kTpk i (consecutive lanes read consecutive pieces of a row).
  // The page of that key is looked up two tiles ahead (lookup), its rows
  // loaded one tile ahead (fetch), so neither load is waited for in the
  // iteration that issues it.
  const int gk = tid / kTpk;
  const int gp = tid % kTpk;
  // Staged rows: 16 bytes (8 fp16) per piece, or 8 bytes (8 int8) and the
  // key's two scales.
  typedef typename std::conditional<Q8, uint2, f16x8>::type piece_t;
  piece_t kr[kPieces], vr[kPieces];
  f16 ksc = (f16)0.0f, vsc = (f16)0.0f;
  bool gok = false;
  // The table read is unconditional (index clamped, table_len >= 1) and its
  // range check a separate flag, so the loaded page id is never merged with
  // another value, which would wait for the load. The cursor (key kp, page
  // index pi, row r in the page) advances one tile per lookup; when the page
  // size divides the tile, r stays fixed and pi steps by a constant.
  int kp = kbase + t_begin * kKeys + gk;
  int pi = kp / p.page_size;
  int r = kp - pi * p.page_size;
  auto lookup = [&](int& page, bool& in, int& row_off, int& scale_off) {
    in = kp <= last && pi < p.table_len;
    page = p.table[min(pi, p.table_len - 1)];
    row_off = r * p.row_elems + kvh * p.head_elems + (GEN ? 0 : gp * 8);
    scale_off = r * p.scale_row + kvh * p.scale_head;
    kp += kKeys;
    if (p.page_step > 0) {
      pi += p.page_step;
    } else {
      pi = kp / p.page_size;
      r = kp - pi * p.page_size;
    }
  };
  // GEN: dim of element pair j of piece i, clamped into the row (pairs past
  // the head dim reload the last pair; trim zeroes them).
  auto pair_dim = [&](int i, int j) { return min(8 * (gp + kTpk * i) + 2 * j, p.head_dim - 2); };
  // ODD: dim of element e of piece i, clamped into the row (elements past
  // the head dim reload the last one; trim zeroes them).
  auto elem_dim = [&](int i, int e) { return min(8 * (gp + kTpk * i) + e, p.head_dim - 1); };
  auto fetch = [&](int page, bool in, int row_off, int scale_off) {
    gok = in && page >= 0 && page < p.arena_pages;
    const uint32_t pg = (uint32_t)(gok ? page : 0);
    const uint64_t at = (uint64_t)pg * (uint64_t)p.page_elems + row_off;
    if constexpr (ODD && Q8) {
      const uint8_t* kb = static_cast<const uint8_t*>(p.k) + at;
      const uint8_t* vb = static_cast<const uint8_t*>(p.v) + at;
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        uint32_t kw[2] = {0u, 0u}, vw[2] = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kw[e / 4] |= (uint32_t)kb[elem_dim(i, e)] << (8 * (e % 4));
          vw[e / 4] |= (uint32_t)vb[elem_dim(i, e)] << (8 * (e % 4));
        }
        kr[i] = uint2{kw[0], kw[1]};
        vr[i] = uint2{vw[0], vw[1]};
      }
      const uint64_t sat = (uint64_t)pg * (uint64_t)p.scale_page + scale_off;
      ksc = p.kscale[sat];
      vsc = p.vscale[sat];
    } else if constexpr (ODD) {
      const uint16_t* kb = reinterpret_cast<const uint16_t*>(static_cast<const f16*>(p.k) + at);
      const uint16_t* vb = reinterpret_cast<const uint16_t*>(static_cast<const f16*>(p.v) + at);
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        i32x4 kw, vw;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kw[j] = (int)((uint32_t)kb[elem_dim(i, 2 * j)] | (uint32_t)kb[elem_dim(i, 2 * j + 1)] << 16);
          vw[j] = (int)((uint32_t)vb[elem_dim(i, 2 * j)] | (uint32_t)vb[elem_dim(i, 2 * j + 1)] << 16);
        }
        kr[i] = __builtin_bit_cast(f16x8, kw);
        vr[i] = __builtin_bit_cast(f16x8, vw);
      }
    } else if constexpr (GEN && Q8) {
      const uint8_t* kb = static_cast<const uint8_t*>(p.k) + at;
      const uint8_t* vb = static_cast<const uint8_t*>(p.v) + at;
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        uint32_t kw[4], vw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kw[j] = *reinterpret_cast<const uint16_t*>(kb + pair_dim(i, j));
          vw[j] = *reinterpret_cast<const uint16_t*>(vb + pair_dim(i, j));
        }
        kr[i] = uint2{kw[0] | kw[1] << 16, kw[2] | kw[3] << 16};
        vr[i] = uint2{vw[0] | vw[1] << 16, vw[2] | vw[3] << 16};
      }
      const uint64_t sat = (uint64_t)pg * (uint64_t)p.scale_page + scale_off;
      ksc = p.kscale[sat];
      vsc = p.vscale[sat];
    } else if constexpr (GEN) {
      const f16* kb = static_cast<const f16*>(p.k) + at;
      const f16* vb = static_cast<const f16*>(p.v) + at;
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        i32x4 kw, vw;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kw[j] = *reinterpret_cast<const int*>(kb + pair_dim(i, j));
          vw[j] = *reinterpret_cast<const int*>(vb + pair_dim(i, j));
        }
        kr[i] = __builtin_bit_cast(f16x8, kw);
        vr[i] = __builtin_bit_cast(f16x8, vw);
      }
    } else if constexpr (Q8) {
      const uint8_t* kb = static_cast<const uint8_t*>(p.k) + at;
      const uint8_t* vb = static_cast<const uint8_t*>(p.v) + at;
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        kr[i] = *reinterpret_cast<const uint2*>(kb + 8 * kTpk * i);
        vr[i] = *reinterpret_cast<const uint2*>(vb + 8 * kTpk * i);
      }
      const uint64_t sat = (uint64_t)pg * (uint64_t)p.scale_page + scale_off;
      ksc = p.kscale[sat];
      vsc = p.vscale[sat];
    } else {
      const f16* kb = static_cast<const f16*>(p.k) + at;
      const f16* vb = static_cast<const f16*>(p.v) + at;
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        kr[i] = *reinterpret_cast<const f16x8*>(kb + 8 * kTpk * i);
        vr[i] = *reinterpret_cast<const f16x8*>(vb + 8 * kTpk * i);
      }
    }
  };
  // A staged piece as 8 fp16 values (8-bit: fp16(int8 x scale), one
  // rounding of the exact product).
  auto as_f16 = [&](const piece_t& x, f16 scale, int i) -> f16x8 {
    f16x8 y;
    if constexpr (Q8) {
      const f16x2 s2 = {scale, scale};
      const uint32_t lo = x.x ^ 0x80808080u, hi = x.y ^ 0x80808080u;
      const f16x2 e0 = pda_internal::bytes_to_f16x2(lo, 0x04010400u) * s2;
      const f16x2 e1 = pda_internal::bytes_to_f16x2(lo, 0x04030402u) * s2;
      const f16x2 e2 = pda_internal::bytes_to_f16x2(hi, 0x04010400u) * s2;
      const f16x2 e3 = pda_internal::bytes_to_f16x2(hi, 0x04030402u) * s2;
      y = f16x8{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
    } else {
      (void)scale;
      y = x;
    }
    if constexpr (ODD) {  // zero the elements past the head dim
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = 8 * (gp + kTpk * i) + e < p.head_dim ? y[e] : (f16)0.0f;
    } else if constexpr (GEN) {  // zero the pairs past the head dim
      i32x4 w4 = __builtin_bit_cast(i32x4, y);
#pragma unroll
      for (int j = 0; j < 4; ++j) w4[j] = 8 * (gp + kTpk * i) + 2 * j < p.head_dim ? w4[j] : 0;
      y = __builtin_bit_cast(f16x8, w4);
    }
    return y;
  };
  auto stash_v = [&](int vbuf) {
    f16* vd = s_v[vbuf] + gk * kVRow + gp * 8;
    if (__ballot(gok) == ~0ull) {
#pragma unroll
      for (int i = 0; i < kPieces; ++i)
        *reinterpret_cast<f16x8*>(vd + 8 * kTpk * i) = as_f16(vr[i], vsc, i);
    } else {
#pragma unroll
      for (int i = 0; i < kPieces; ++i)
        *reinterpret_cast<f16x8*>(vd + 8 * kTpk * i) = gok ? as_f16(vr[i], vsc, i) : f16x8{};
    }
  };
  auto stash = [&](int buf) {
    // Unusable keys are stored as zeros (their weight is 0; zero V keeps
    // 0 * V finite whatever the arena holds there).
    f16* kd = s_k[buf] + gk * kKRow + gp * 8;
    const uint64_t bits = __ballot(gok);
    if constexpr (kOneV) {
#pragma unroll
      for (int i = 0; i < kPieces; ++i)
        *reinterpret_cast<f16x8*>(kd + 8 * kTpk * i) = gok ? as_f16(kr[i], ksc, i) : f16x8{};
    } else {
      f16* vd = s_v[buf] + gk * kVRow + gp * 8;
      if (bits == ~0ull) {  // wave-uniform: the usual case stores without selects
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
          *reinterpret_cast<f16x8*>(kd + 8 * kTpk * i) = as_f16(kr[i], ksc, i);
          *reinterpret_cast<f16x8*>(vd + 8 * kTpk * i) = as_f16(vr[i], vsc, i);
        }
      } else {
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
          *reinterpret_cast<f16x8*>(kd + 8 * kTpk * i) = gok ? as_f16(kr[i], ksc, i) : f16x8{};
          *reinterpret_cast<f16x8*>(vd + 8 * kTpk * i) = gok ? as_f16(vr[i], vsc, i) : f16x8{};
        }
      }
    }
    if (lane == 0) {
      uint32_t mk = 0;
#pragma unroll
      for (int j = 0; j < kKeysPerWave; ++j) mk |= (uint32_t)((bits >> (kTpk * j)) & 1) << j;
      s_ok[buf][w] = (okbits)mk;
    }
  };

  // Lane part of the transposed V read: group g = lane / 16 reads dims
  // 16 (g % 2) + 4 (s % 4) of key 4 (g / 2) + s / 4, s = lane % 16.
  const int g16 = lane >> 4, s16 = lane & 15;
  const int v_lane =
      (4 * (g16 >> 1) + (s16 >> 2)) * kVRow + 16 * (g16 & 1) + 4 * (s16 & 3) + sl * kDW;
  const int k_lane = n * kKRow + 8 * hh + sl * kDW;
  const int qlo = p.window > 0 ? qpos - p.window : INT32_MIN;  // keys > qlo are in the window
  const float c = p.softcap <= 0.0f && p.scale_log2 > 0.0f ? p.scale_log2 : 1.0f;

  int page0, r0, s0, page1, r1, s1;
  bool in0, in1;
  lookup(page0, in0, r0, s0);
  lookup(page1, in1, r1, s1);
  fetch(page0, in0, r0, s0);
  stash(0);
  if constexpr (kOneV) stash_v(0);
  __syncthreads();
  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1;
    const int k0 = kbase + t * kKeys;
    const bool more = t + 1 < t_end;
    // V of this tile, staged in the previous iteration (every wave finished
    // that tile's V at its closing barrier; the score exchange's barrier
    // below publishes these stores before any wave reads them).
    if constexpr (kOneV)
      if (t > t_begin) stash_v(0);
    if (more) fetch(page1, in1, r1, s1);
    lookup(page1, in1, r1, s1);

    const bool work = wave_live && k0 <= wave_last &&
                      (p.window <= 0 || wave_img || k0 + kKeys - 1 > wfirst - p.window);
    const f16* sk = s_k[buf];
    const f16* sv = s_v[kOneV ? 0 : buf];
    // S^T per 32-key block kb: lane holds keys 32 kb + 8 (v / 4) + 4 hh + v % 4.
    f32x16 s[KB];
    if (work) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        f16x8 ka[kDW / 16];
#pragma unroll
        for (int c = 0; c < kDW / 16; ++c)
          ka[c] = *reinterpret_cast<const f16x8*>(sk + k_lane + 32 * kb * kKRow + 16 * c);
        s[kb] = f32x16{};
        // Raised wave priority while this wave issues matrix-core work: the
        // SIMD's other wave, in its softmax, then yields the issue slots and
        // the matrix core is fed while the VALU phase of one wave overlaps
        // the MFMA phase of the other (2-4% on config 2's chunks).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int c = 0; c < kDW / 16; ++c)
          s[kb] = mfma16<BF>(ka[c], qf[c], s[kb]);
        __builtin_amdgcn_s_setprio(0);
      }
    }
    if constexpr (kSlices > 1) {
      // Sum the slices' partial scores in slice order, so that every wave of
      // the block holds the same scores, maximum, sum and probabilities.
      // `work` is the same for all of them (it depends on the queries only).
      // Reduce-scatter then gather: 12 adds per lane instead of 48. Slice sl
      // sums groups [sl kPer, (sl + 1) kPer) of the block's partials in
      // slice order; then every wave reads all the sums.
      if (work) {
#pragma unroll
        for (int i = 0; i < kGroups; ++i)
          s_x[w * kGroups + i][lane] = make_float4(s[i / 4][4 * (i % 4)], s[i / 4][4 * (i % 4) + 1],
                                                   s[i / 4][4 * (i % 4) + 2],
                                                   s[i / 4][4 * (i % 4) + 3]);
      }
      __syncthreads();
      if (work) {
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
          const int i = sl * kPer + r;
          float4 acc = s_x[qb * kSlices * kGroups + i][lane];
#pragma unroll
          for (int j = 1; j < kSlices; ++j) {
            const float4 y = s_x[(qb * kSlices + j) * kGroups + i][lane];
            acc.x += y.x;
            acc.y += y.y;
            acc.z += y.z;
            acc.w += y.w;
          }
          s_y[w * kPer + r][lane] = acc;
        }
      }
      __syncthreads();
      if (work) {
#pragma unroll
        for (int i = 0; i < kGroups; ++i) {
          const float4 acc = s_y[(qb * kSlices + i / kPer) * kPer + i % kPer][lane];
          s[i / 4][4 * (i % 4)] = acc.x;
          s[i / 4][4 * (i % 4) + 1] = acc.y;
          s[i / 4][4 * (i % 4) + 2] = acc.z;
          s[i / 4][4 * (i % 4) + 3] = acc.w;
        }
      }
    }
    if (work) {
      okword okm;
      if constexpr (kKeysPerWave == 4) {
        // Eight waves of four keys: one nibble per byte, packed to 32 bits.
        uint64_t x = *reinterpret_cast<const uint64_t*>(s_ok[buf]) & 0x0F0F0F0F0F0F0F0Full;
        x = (x | (x >> 4)) & 0x00FF00FF00FF00FFull;
        x = (x | (x >> 8)) & 0x0000FFFF0000FFFFull;
        okm = (okword)(x | (x >> 16));
      } else {
        okm = *reinterpret_cast<const okword*>(s_ok[buf]);
      }
      const bool edge = k0 + kKeys - 1 > wfirst || okm != (okword)~(okword)0 ||
                        (p.window > 0 && k0 <= wlast - p.window);
      // x = score in units that exp2(x * c - m) turns into the weight: the
      // raw q.k with c = scale log2(e) when that is positive (the max of raw
      // scores gives the max of the scaled ones), else the scaled or
      // softcapped score in log2 units with c = 1.
      float x[16 * KB];
      if (p.softcap > 0.0f) {
#pragma unroll
        for (int v = 0; v < 16 * KB; ++v) {
          const float e = __builtin_amdgcn_exp2f(s[v / 16][v % 16] * p.cap_in);
          x[v] = (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f)) * p.cap_out;
        }
      } else if (p.scale_log2 > 0.0f) {
#pragma unroll
        for (int v = 0; v < 16 * KB; ++v) x[v] = s[v / 16][v % 16];
      } else {
#pragma unroll
        for (int v = 0; v < 16 * KB; ++v) x[v] = s[v / 16][v % 16] * p.scale_log2;
      }
      if (edge) {
        // Key k0 + key is visible to this lane's query when usable,
        // <= qpos and > qlo.
        const okword okl = okm >> (4 * hh);
        const int hi = qpos - k0 - 4 * hh;  // largest visible key offset
        const int lo = qlo == INT32_MIN ? INT32_MIN : qlo - k0 - 4 * hh;
        const int ilo = img_lo - k0 - 4 * hh, ihi = img_hi - k0 - 4 * hh;  // image span
        // Bitwise operators, not && / ||: the short-circuit form compiled to
        // nested exec-mask branches, one of which dropped the restore of the
        // score for lanes visible through the image span only.
#pragma unroll
        for (int v = 0; v < 16 * KB; ++v) {
          const int key = 32 * (v / 16) + 8 * ((v % 16) / 4) + (v % 4);  // minus 4 hh
          const bool usable_key = ((okl >> key) & 1u) != 0;
          const bool causal = (key <= hi) & (key > lo);
          const bool image = (key >= ilo) & (key < ihi);
          x[v] = usable_key & (causal | image) ? x[v] : -INFINITY;
        }
      }
      // Lazy running max: rescale only when a score passes it by 2^8.
      // Returns whether this lane's max moved.
      auto lazy_max = [&]() -> bool {
        float top = x[0];
#pragma unroll
        for (int v = 1; v < 16 * KB; ++v) top = fmaxf(top, x[v]);
        top = fmaxf(top, __shfl_xor(top, 32)) * c;  // with the other half of this query's keys
        if (top > m + kSlack) {
          const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - top);
          m = top;
          l *= f;
#pragma unroll
          for (int b = 0; b < kDW / 32; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[b][v] *= f;
          return true;
        }
        return false;
      };
      // P^T as the B operand: 16-key step ks holds values 8 ks .. 8 ks + 7,
      // i.e. keys 16 ks + 8 (t / 4) + 4 hh + t % 4. O^T += V^T P^T, A
      // operand of step ks for rows 32 b ..: keys 16 ks + 4 hh + 0..3 (first
      // read) and + 8 (second read).
      f16x8 pb[2 * KB];
      // The weights exp2(x c - mu) as 16-bit B operands, summed into `sum`.
      auto weights = [&](float mu, float& sum) {
#pragma unroll
        for (int ks = 0; ks < 2 * KB; ++ks) {
#pragma unroll
          for (int t2 = 0; t2 < 4; ++t2) {
            if constexpr (BF) {
              const bf16x2 pp = {(bf16)__builtin_amdgcn_exp2f(fmaf(x[8 * ks + 2 * t2], c, -mu)),
                                 (bf16)__builtin_amdgcn_exp2f(fmaf(x[8 * ks + 2 * t2 + 1], c, -mu))};
              sum = __builtin_amdgcn_fdot2_f32_bf16(pp, bf16x2{(bf16)1.0f, (bf16)1.0f}, sum, false);
              const f16x2 ph = __builtin_bit_cast(f16x2, pp);
              pb[ks][2 * t2] = ph[0];
              pb[ks][2 * t2 + 1] = ph[1];
            } else {
              const f16x2 ph = {(f16)__builtin_amdgcn_exp2f(fmaf(x[8 * ks + 2 * t2], c, -mu)),
                                (f16)__builtin_amdgcn_exp2f(fmaf(x[8 * ks + 2 * t2 + 1], c, -mu))};
              sum = __builtin_amdgcn_fdot2(ph, f16x2{(f16)1.0f, (f16)1.0f}, sum, false);
              pb[ks][2 * t2] = ph[0];
              pb[ks][2 * t2 + 1] = ph[1];
            }
          }
        }
      };
      // Optimistic weights (every width but 128): the weights against the
      // running max first. A weight past 2^8 (the lazy max's bound, which
      // keeps 16-bit weights finite) makes the lane's weights sum past 2^8;
      // only then, or while the lane's max is still -inf (every key so far
      // masked, or none seen), does the wave take the max, and weigh again
      // where it moved. (At D = 512 the four slices of a query block hold
      // the same scores, so they decide alike.) The max's reduction chain
      // leaves the common path: 3-7% faster at D = 64, 2-5% at D = 256, 2%
      // at D = 96, 1.3-2.4% at D = 512 (there against issuing each 16-key
      // step's products as soon as its probabilities exist, max first); at
      // D = 128 0-3% slower on causal prompts, so it keeps the max first.
      constexpr bool kOptimistic = D != 128;
      if constexpr (!kOptimistic) {
        lazy_max();
        // While every key so far is masked, m is -inf and so is every x.
        weights(m == -INFINITY ? 0.0f : m, l);
      } else {
        float lb = 0.0f;
        weights(m == -INFINITY ? 0.0f : m, lb);
        if (__ballot(m == -INFINITY || !(lb <= 256.0f)) != 0) {
          if (__ballot(lazy_max()) != 0) {
            lb = 0.0f;
            weights(m == -INFINITY ? 0.0f : m, lb);
          }
        }
        l += lb;
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int b = 0; b < kDW / 32; ++b) {
#pragma unroll
        for (int ks = 0; ks < 2 * KB; ++ks) {
          const f16* vp = sv + v_lane + 16 * ks * kVRow + 32 * b;
          const f16x4 lo4 = read_tr(vp);
          const f16x4 hi4 = read_tr(vp + 8 * kVRow);
          const f16x8 a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          o[b] = mfma16<BF>(a, pb[ks], o[b]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
    if (more) stash(buf ^ 1);
    __syncthreads();  // the next tile is in LDS; this one may be overwritten
  }

  if (!q_live) return;
  l += __shfl_xor(l, 32);
  if (p.splits > 1) {
    // Unnormalised partial and its (max, sum) for the merge; an empty or
    // fully masked range leaves m = -inf, l = 0 and zeros.
    const int64_t at = ((int64_t)split * p.count + qi) * p.hq + h;  // partials are D wide
    float* dst = p.part_o + at * D + sl * kDW;
#pragma unroll
    for (int b = 0; b < kDW / 32; ++b)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(dst + 32 * b + 8 * g + 4 * hh) =
            make_float4(o[b][4 * g], o[b][4 * g + 1], o[b][4 * g + 2], o[b][4 * g + 3]);
    if (hh == 0 && sl == 0) p.part_ml[at] = make_float2(m, l);
    return;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if constexpr (ODD) {
    // Rows of an odd number of elements: one element per store.
    const int hd = p.head_dim;
    f16* dst = p.out + ((int64_t)qi * p.hq + h) * hd;
#pragma unroll
    for (int b = 0; b < kDW / 32; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int d = sl * kDW + 32 * b + 8 * (v / 4) + 4 * hh + v % 4;
        if (d < hd) dst[d] = round16<BF>(o[b][v] * inv);
      }
    return;
  }
  if constexpr (GEN) {
    // Rows of head_dim elements: element pairs, the real dims only.
    const int hd = p.head_dim;
    f16* dst = p.out + ((int64_t)qi * p.hq + h) * hd;
#pragma unroll
    for (int b = 0; b < kDW / 32; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = sl * kDW + 32 * b + 8 * g + 4 * hh;
        const f16x2 y0 = {round16<BF>(o[b][4 * g] * inv), round16<BF>(o[b][4 * g + 1] * inv)};
        const f16x2 y1 = {round16<BF>(o[b][4 * g + 2] * inv),
                          round16<BF>(o[b][4 * g + 3] * inv)};
        if (d < hd) *reinterpret_cast<f16x2*>(dst + d) = y0;
        if (d + 2 < hd) *reinterpret_cast<f16x2*>(dst + d + 2) = y1;
      }
    }
    return;
  }
  f16* dst = p.out + ((int64_t)qi * p.hq + h) * D + sl * kDW;
  // O^T rows: element 32 b + 8 (v / 4) + 4 hh + v % 4 of query n (of the slice).
#pragma unroll
  for (int b = 0; b < kDW / 32; ++b) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f16x4 y;
#pragma unroll
      for (int t = 0; t < 4; ++t) y[t] = round16<BF>(o[b][4 * g + t] * inv);
      *reinterpret_cast<f16x4*>(dst + 32 * b + 8 * g + 4 * hh) = y;
    }
  }
}

// The prefill kernel of every even head dim (template arguments as
// prefill_body's).
template <int D, bool Q8, bool BF, bool GEN>
__global__ __launch_bounds__(64 * waves_for(D)) void paged_prefill_kernel(const PrefillParams p) {
  prefill_body<D, Q8, BF, GEN, false>(p);
}

// Odd head dims (the reference's portable attention takes any): the generic
// kernel of width D with element-wise queries, gather and output.
template <int D, bool Q8, bool BF>
__global__ __launch_bounds__(64 * waves_for(D)) void paged_prefill_odd_kernel(const PrefillParams p) {
  prefill_body<D, Q8, BF, true, true>(p);
}

// Merge of the key ranges of a split prefill: for each (query, head),
// M = max_s m_s, w_s = 2^(m_s - M) (0 for an empty range), out =
// sum_s w_s o_s / sum_s w_s l_s (0 when nothing was visible). The same LSE
// merge as the reference's decode merge (metal_kernels.py:103-124), in the
// log2 domain. One thread per 4 dims, D / 4 threads per (query, head).
// GEN: output rows of hd (below D) elements, written one element at a time
// (an odd hd leaves rows 2-byte aligned); partials stay D wide.
template <int D, bool BF, bool GEN>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float* __restrict__ part_o,
                                                            const float2* __restrict__ part_ml,
                                                            f16* __restrict__ out, int64_t pairs,
                                                            int splits, int hd) {
  constexpr int kT = D / 4;
  // 256 / kT pairs per block; at D = 96 the last 16 threads have none.
  if (threadIdx.x >= 256 / kT * kT) return;
  const int64_t pair = (int64_t)blockIdx.x * (256 / kT) + threadIdx.x / kT;
  if (pair >= pairs) return;
  const int d = 4 * (threadIdx.x % kT);
  float top = -INFINITY;
  for (int s = 0; s < splits; ++s) top = fmaxf(top, part_ml[s * pairs + pair].x);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float sum = 0.0f;
  if (top != -INFINITY) {
    for (int s = 0; s < splits; ++s) {
      const float2 ml = part_ml[s * pairs + pair];
      if (ml.x == -INFINITY) continue;
      const float w = __builtin_amdgcn_exp2f(ml.x - top);
      const float4 x = *reinterpret_cast<const float4*>(part_o + (s * pairs + pair) * D + d);
      acc.x += w * x.x;
      acc.y += w * x.y;
      acc.z += w * x.z;
      acc.w += w * x.w;
      sum += w * ml.y;
    }
  }
  const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
  f16x4 y = {round16<BF>(acc.x * inv), round16<BF>(acc.y * inv), round16<BF>(acc.z * inv),
             round16<BF>(acc.w * inv)};
  if constexpr (GEN) {
    f16* row = out + pair * hd;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (d + j < hd) row[d + j] = y[j];
  } else {
    (void)hd;
    *reinterpret_cast<f16x4*>(out + pair * D + d) = y;
  }
}

constexpr int kCus = 256;       // MI355X compute units
constexpr int kMaxSplits = 64;

// Key ranges per (query tile, head): 1 when the tiles and heads alone give
// every workgroup slot of the GPU (CUs x the kernel's occupancy) its work,
// else as many as fit the slots in one round: the ranges of a chunk over a
// long prefix are all alike, so a partly filled second round would cost a
// whole range's time. One exception: a causal chunk that fills at most one
// round and whose first query tile sees at most half the keys of its last
// (a prompt from position 0) takes 2 ranges, so that the halves of its
// longest tiles run beside its short ones. Each range holds at least 8 key
// tiles. `request` > 0 forces a count.
int prefill_splits(int start, int count, int q_heads, int head_dim, int window, int request) {
  if (request > 0) return request < kMaxSplits ? request : kMaxSplits;
  const int queries = queries_for(head_dim);
  const int64_t wgs = (int64_t)(count + queries - 1) / queries * q_heads;
  const int occupancy = head_dim == 64 ? 3 : head_dim <= 128 ? 2 : 1;
  const int64_t slots = (int64_t)kCus * occupancy;
  const int keys = 32 * (head_dim <= 128 ? 2 : 1);
  // Keys seen by the chunk's first and last query tiles.
  const int64_t cap = window > 0 ? (int64_t)window + queries : INT64_MAX;
  const int64_t first = std::min<int64_t>((int64_t)start + std::min(count, queries), cap);
  const int64_t span = std::min<int64_t>((int64_t)start + count, cap);
  const int64_t by_keys = (span + keys - 1) / keys / 8;
  if (wgs * 2 > slots) return wgs <= slots && 2 * first <= span && by_keys >= 2 ? 2 : 1;
  int64_t s = slots / wgs;
  if (s > by_keys) s = by_keys;
  if (s > kMaxSplits) s = kMaxSplits;
  return s < 1 ? 1 : (int)s;
}

size_t prefill_workspace(int splits, int count, int q_heads, int head_dim) {
  if (splits <= 1) return 0;
  const size_t pairs = (size_t)count * q_heads;
  // Partial outputs, then the (max, sum) pairs, each 256-byte aligned.
  const size_t o_bytes = ((size_t)splits * pairs * head_dim * 4 + 255) & ~(size_t)255;
  return o_bytes + (((size_t)splits * pairs * 8 + 255) & ~(size_t)255);
}

using pda_internal::fail;
using pda_internal::ok;

// The kernel width serving a head dim: the head dim itself when a kernel
// has it, else the next wider one (GEN kernels; odd head dims the odd
// kernels); 0 for head dims the library does not serve (above 512).
int prefill_dim(int head_dim) {
  if (head_dim < 1 || head_dim > 512) return 0;
  for (int d : {64, 96, 128, 256, 512})
    if (head_dim <= d) return d;
  return 0;
}

template <bool Q8, bool BF, bool GEN>
const void* prefill_kernel_for(int kdim) {
  return kdim == 64    ? reinterpret_cast<const void*>(paged_prefill_kernel<64, Q8, BF, GEN>)
         : kdim == 96  ? reinterpret_cast<const void*>(paged_prefill_kernel<96, Q8, BF, GEN>)
         : kdim == 128 ? reinterpret_cast<const void*>(paged_prefill_kernel<128, Q8, BF, GEN>)
         : kdim == 256 ? reinterpret_cast<const void*>(paged_prefill_kernel<256, Q8, BF, GEN>)
                       : reinterpret_cast<const void*>(paged_prefill_kernel<512, Q8, BF, GEN>);
}

template <bool Q8, bool BF>
const void* prefill_odd_kernel_for(int kdim) {
  return kdim == 64    ? reinterpret_cast<const void*>(paged_prefill_odd_kernel<64, Q8, BF>)
         : kdim == 96  ? reinterpret_cast<const void*>(paged_prefill_odd_kernel<96, Q8, BF>)
         : kdim == 128 ? reinterpret_cast<const void*>(paged_prefill_odd_kernel<128, Q8, BF>)
         : kdim == 256 ? reinterpret_cast<const void*>(paged_prefill_odd_kernel<256, Q8, BF>)
                       : reinterpret_cast<const void*>(paged_prefill_odd_kernel<512, Q8, BF>);
}

template <bool Q8, bool BF>
const void* prefill_kernel_for(int kdim, bool gen, bool odd) {
  if (odd) return prefill_odd_kernel_for<Q8, BF>(kdim);
  return gen ? prefill_kernel_for<Q8, BF, true>(kdim) : prefill_kernel_for<Q8, BF, false>(kdim);
}

template <bool BF, bool GEN>
const void* merge_kernel_for(int kdim) {
  return kdim == 64    ? reinterpret_cast<const void*>(prefill_merge_kernel<64, BF, GEN>)
         : kdim == 96  ? reinterpret_cast<const void*>(prefill_merge_kernel<96, BF, GEN>)
         : kdim == 128 ? reinterpret_cast<const void*>(prefill_merge_kernel<128, BF, GEN>)
         : kdim == 256 ? reinterpret_cast<const void*>(prefill_merge_kernel<256, BF, GEN>)
                       : reinterpret_cast<const void*>(prefill_merge_kernel<512, BF, GEN>);
}

template <bool BF>
const void* merge_kernel_for(int kdim, bool gen) {
  return gen ? merge_kernel_for<BF, true>(kdim) : merge_kernel_for<BF, false>(kdim);
}

int prefill(const void* queries, const void* keys, const void* values, const void* key_scales,
            const void* value_scales, bool q8, bool bf16_elems, const int32_t* table,
            int32_t table_len,
            int32_t start, int32_t count, void* out, int32_t q_heads, int32_t kv_heads,
            int32_t head_dim, int32_t page_size, int64_t arena_rows, int32_t layout, float scale,
            int32_t window, float softcap, const int32_t* images, int32_t num_images,
            int32_t splits, void* workspace, size_t workspace_bytes, void* stream) {
  if (count < 0 || start < 0 || q_heads <= 0 || kv_heads <= 0 || page_size <= 0 ||
      table_len < 0 || window < 0 || splits < 0)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "count=%d start=%d q_heads=%d kv_heads=%d page_size=%d table_len=%d window=%d "
                "splits=%d",
                count, start, q_heads, kv_heads, page_size, table_len, window, splits);
  if (q_heads % kv_heads)
    return fail(PDA_ERR_HEAD_RATIO, "query heads must be a multiple of kv heads");
  const int kdim = prefill_dim(head_dim);
  if (kdim == 0)
    return fail(PDA_ERR_HEAD_DIM, "head_dim %d: prefill serves head dims 1..512", head_dim);
  const bool gen = kdim != head_dim;
  const bool odd = head_dim & 1;
  if (count == 0) return ok();
  if (table_len == 0)
    return fail(PDA_ERR_INVALID_ARGUMENT, "an empty page table holds no keys of the chunk");
  if ((int64_t)start + count > INT32_MAX)
    return fail(PDA_ERR_TOO_LONG, "start + count exceeds 2^31");
  if (!queries || !keys || !values || !table || !out || (q8 && (!key_scales || !value_scales)))
    return fail(PDA_ERR_INVALID_ARGUMENT, "null buffer pointer");
  if (num_images < 0 || (num_images > 0 && !images))
    return fail(PDA_ERR_INVALID_ARGUMENT, "num_images=%d needs an image span array",
                num_images);
  if ((uintptr_t)images & 3) return fail(PDA_ERR_ALIGNMENT, "image spans must be 4-byte aligned");
  if (layout != PDA_LAYOUT_ROWS && layout != PDA_LAYOUT_PAGES)
    return fail(PDA_ERR_INVALID_ARGUMENT, "unknown K/V layout %d", layout);
  if ((int64_t)page_size * kv_heads * head_dim > INT32_MAX)
    return fail(PDA_ERR_INVALID_ARGUMENT, "a page of one layer holds more than 2^31 elements");
  if (arena_rows < page_size)
    return fail(PDA_ERR_INVALID_ARGUMENT, "arena_rows %lld holds no whole page",
                (long long)arena_rows);
  if (!(scale == scale) || isinf(scale) || !(softcap >= 0.0f) || isinf(softcap))
    return fail(PDA_ERR_INVALID_ARGUMENT, "scale must be finite and softcap >= 0");
  const uintptr_t mis = (uintptr_t)queries | (uintptr_t)keys | (uintptr_t)values |
                        (uintptr_t)out;
  if (mis & 15)
    return fail(PDA_ERR_ALIGNMENT, "query, K/V and output buffers must be 16-byte aligned");
  if (q8 && (((uintptr_t)key_scales | (uintptr_t)value_scales) & 1))
    return fail(PDA_ERR_ALIGNMENT, "fp16 scale arenas must be 2-byte aligned");
  if ((uintptr_t)table & 3) return fail(PDA_ERR_ALIGNMENT, "the table must be 4-byte aligned");
  const int nsplit = prefill_splits(start, count, q_heads, kdim, window, splits);
  const int per_wg = queries_for(kdim);
  if ((int64_t)((count + per_wg - 1) / per_wg) * q_heads * nsplit > INT32_MAX)
    return fail(PDA_ERR_INVALID_ARGUMENT, "query tiles x query heads x splits exceeds 2^31");
  const size_t need = prefill_workspace(nsplit, count, q_heads, kdim);
  if (need > 0 && (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255)))
    return fail(PDA_ERR_WORKSPACE,
                "%d key ranges need a 256-byte aligned workspace of %zu bytes (got %zu)", nsplit,
                need, workspace ? workspace_bytes : (size_t)0);

  PrefillParams prm;
  prm.q = static_cast<const f16*>(queries);
  prm.k = keys;
  prm.v = values;
  prm.kscale = static_cast<const f16*>(key_scales);
  prm.vscale = static_cast<const f16*>(value_scales);
  // Scale arenas: [rows, kv_heads] beside the row arena, [pages, kv_heads,
  // page_size] beside page tiles (as the decode call's).
  prm.scale_page = (int64_t)page_size * kv_heads;
  prm.scale_row = layout == PDA_LAYOUT_ROWS ? kv_heads : 1;
  prm.scale_head = layout == PDA_LAYOUT_ROWS ? 1 : page_size;
  prm.table = table;
  prm.images = images;
  prm.num_images = num_images;
  prm.out = static_cast<f16*>(out);
  const size_t pairs = (size_t)count * q_heads;
  prm.part_o = nsplit > 1 ? static_cast<float*>(workspace) : nullptr;
  prm.part_ml = nsplit > 1 ? reinterpret_cast<float2*>(
                                 static_cast<char*>(workspace) +
                                 (((size_t)nsplit * pairs * kdim * 4 + 255) & ~(size_t)255))
                           : nullptr;
  prm.arena_pages = arena_rows / page_size;
  prm.page_elems = (int64_t)page_size * kv_heads * head_dim;
  if (layout == PDA_LAYOUT_ROWS) {
    prm.row_elems = kv_heads * head_dim;
    prm.head_elems = head_dim;
  } else {
    prm.row_elems = head_dim;
    prm.head_elems = page_size * head_dim;
  }
  prm.table_len = table_len;
  prm.start = start;
  prm.count = count;
  prm.tiles = (count + per_wg - 1) / per_wg;
  prm.splits = nsplit;
  const int tile_keys = kdim <= 128 ? 64 : 32;
  prm.page_step = tile_keys % page_size == 0 ? tile_keys / page_size : 0;
  prm.hq = q_heads;
  prm.hkv = kv_heads;
  prm.head_dim = head_dim;
  prm.page_size = page_size;
  prm.window = window;
  prm.scale_log2 = scale * kLog2e;
  prm.softcap = softcap;
  prm.cap_in = softcap > 0.0f ? 2.0f * kLog2e * scale / softcap : 0.0f;
  prm.cap_out = softcap * kLog2e;
  void* args[] = {&prm};
  const void* fn = q8 ? prefill_kernel_for<true, false>(kdim, gen, odd)
                  : bf16_elems ? prefill_kernel_for<false, true>(kdim, gen, odd)
                               : prefill_kernel_for<false, false>(kdim, gen, odd);
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((int64_t)prm.tiles * q_heads * nsplit));
  hipError_t err = hipLaunchKernel(fn, grid, dim3(64 * waves_for(kdim)), args, 0, hs);
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  if (nsplit > 1) {
    const int64_t npairs = (int64_t)pairs;
    const int per_block = 256 / (kdim / 4);
    const float* po = prm.part_o;
    const float2* pml = prm.part_ml;
    f16* o16 = prm.out;
    int ns = nsplit;
    int hd = head_dim;
    void* margs[] = {&po, &pml, &o16, (void*)&npairs, &ns, &hd};
    const void* mfn = bf16_elems ? merge_kernel_for<true>(kdim, gen)
                                 : merge_kernel_for<false>(kdim, gen);
    err = hipLaunchKernel(mfn, dim3((unsigned)((npairs + per_block - 1) / per_block)),
                          dim3(256), margs, 0, hs);
    if (err != hipSuccess)
      return fail(PDA_ERR_HIP, "merge launch failed: %s", hipGetErrorString(err));
  }
  return ok();
}

}  // namespace

extern "C" {

int pda_prefill_workspace_bytes(int32_t start, int32_t count, int32_t q_heads,
                                int32_t head_dim, int32_t window, int32_t splits,
                                int32_t* splits_used, size_t* bytes) {
  if (count < 0 || start < 0 || q_heads <= 0 || window < 0 || splits < 0 || !bytes)
    return fail(PDA_ERR_INVALID_ARGUMENT, "count=%d start=%d q_heads=%d window=%d splits=%d",
                count, start, q_heads, window, splits);
  const int kdim = prefill_dim(head_dim);
  if (kdim == 0)
    return fail(PDA_ERR_HEAD_DIM, "head_dim %d: prefill serves head dims 1..512", head_dim);
  const int s = count == 0 ? 1 : prefill_splits(start, count, q_heads, kdim, window, splits);
  if (splits_used) *splits_used = s;
  *bytes = prefill_workspace(s, count, q_heads, kdim);
  return ok();
}

int pda_paged_prefill_attention(const void* queries, const void* keys, const void* values,
                                const int32_t* table, int32_t table_len, int32_t start,
                                int32_t count, void* out, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, int32_t page_size, int64_t arena_rows,
                                int32_t layout, float scale, int32_t window, float softcap,
                                const int32_t* images, int32_t num_images, int32_t splits,
                                void* workspace, size_t workspace_bytes, void* stream) {
  return prefill(queries, keys, values, nullptr, nullptr, false, false, table, table_len, start,
                 count, out, q_heads, kv_heads, head_dim, page_size, arena_rows, layout, scale,
                 window, softcap, images, num_images, splits, workspace, workspace_bytes, stream);
}

int pda_paged_prefill_attention_bf16(const void* queries, const void* keys, const void* values,
                                     const int32_t* table, int32_t table_len, int32_t start,
                                     int32_t count, void* out, int32_t q_heads,
                                     int32_t kv_heads, int32_t head_dim, int32_t page_size,
                                     int64_t arena_rows, int32_t layout, float scale,
                                     int32_t window, float softcap, const int32_t* images,
                                     int32_t num_images, int32_t splits, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return prefill(queries, keys, values, nullptr, nullptr, false, true, table, table_len, start,
                 count, out, q_heads, kv_heads, head_dim, page_size, arena_rows, layout, scale,
                 window, softcap, images, num_images, splits, workspace, workspace_bytes, stream);
}

int pda_paged_prefill_attention_q8(const void* queries, const void* keys, const void* values,
                                   const void* key_scales, const void* value_scales,
                                   const int32_t* table, int32_t table_len, int32_t start,
                                   int32_t count, void* out, int32_t q_heads, int32_t kv_heads,
                                   int32_t head_dim, int32_t page_size, int64_t arena_rows,
                                   int32_t layout, float scale, int32_t window, float softcap,
                                   const int32_t* images, int32_t num_images, int32_t splits,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  return prefill(queries, keys, values, key_scales, value_scales, true, false, table, table_len,
                 start, count, out, q_heads, kv_heads, head_dim, page_size, arena_rows, layout,
                 scale, window, softcap, images, num_images, splits, workspace, workspace_bytes,
                 stream);
}

}  // extern "C"
