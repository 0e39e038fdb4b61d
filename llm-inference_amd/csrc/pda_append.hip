// K/V append with rotary position embedding for MI355X (gfx950), C-ABI in
// pda.h (pda_rope_append).
//
// Reference steps fused here, per attention layer and decode step:
//   q = batch.rope(q, dims, base | freqs); k = batch.rope(k, ...)
//       (python/instinct/batches.py:195-201 -> backends/portable.py:88-132,
//       the non-traditional "split-half" rotation: element i pairs with
//       i + dims / 2, angle = position * inv_freq[i], computed in float32)
//   cache.write(layer, rows, k, v)
//       (batches.py:203-207 -> paged_kv.py:278-283: scatter the rotated key
//       and the value of each token into arena row rows[t])
// The CUDA engine fuses the same steps (cuda/kernels.cu:123-170).
//
// MI355X design: one wave per (token, head), four per workgroup, so a decode
// batch of 64 tokens still spreads over a few hundred workgroups. Lanes walk
// the rotation pairs of consecutive elements, so every wave instruction
// touches one contiguous run of a head, and each lane computes its own angles
// (sincosf with full range reduction: positions reach 10^5 and more) while
// its source elements load. The arena write goes to either K/V layout (rows or
// page tiles) by the same strides as the decode kernel. The rotation uses
// separately rounded float32 products and sums (no contraction), the order of
// the reference's float32 expression, and rounds to fp16 to nearest even.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "pda.h"
#include "pda_internal.h"

namespace {

typedef _Float16 f16;
typedef __bf16 bf16;

constexpr int kHeadsPerGroup = 4;  // heads of one token per workgroup, one wave each
constexpr int kAppendThreads = 64 * kHeadsPerGroup;
constexpr int kMaxHalf = 256;      // rope_dims / 2 for head_dim <= 512
constexpr int kMaxHeadDim = 2 * kMaxHalf;

struct AppendParams {
  const f16* q;
  f16* q_out;
  const f16* k;
  const f16* v;
  void* k_arena;      // fp16, or int8 with scale arenas (8-bit K/V)
  void* v_arena;
  f16* k_scale;       // 8-bit: fp16 scale per (row, kv head)
  f16* v_scale;
  const int32_t* positions;
  const int32_t* rows;
  const float* inv_freq;
  int64_t arena_rows;
  int32_t hq;        // query heads rotated (0 when q is null)
  int32_t hkv;       // kv heads written (0 when k is null)
  int32_t d;         // head_dim
  int32_t half;      // rope_dims / 2
  int32_t page_size;
  int32_t layout;
};

// Scale of kv head h in arena row `row`: [rows, kv_heads] beside a row arena,
// [pages, kv_heads, page_size] beside a page-tile arena.
__device__ __forceinline__ int64_t scale_index(const AppendParams& p, int64_t row, int h) {
  if (p.layout == PDA_LAYOUT_ROWS) return row * p.hkv + h;
  const int64_t page = row / p.page_size;
  return (page * p.hkv + h) * p.page_size + (row - page * p.page_size);
}

// Element e of kv head h in arena row `row`, in either layout.
__device__ __forceinline__ int64_t arena_index(const AppendParams& p, int64_t row, int h,
                                               int e) {
  if (p.layout == PDA_LAYOUT_ROWS) return (row * p.hkv + h) * p.d + e;
  const int64_t page = row / p.page_size;
  const int64_t slot = row - page * p.page_size;
  return ((page * p.hkv + h) * p.page_size + slot) * p.d + e;
}

// Rotates one head: pairs (j, j + half) for j < half, the elements from
// 2 * half on are copied. Lane `lane` of the head's wave takes j = lane,
// lane + 64, ...; the source elements are loaded before the angles are
// computed, so their latency overlaps the position and frequency loads.
// E: the element type of q, k and the arena (fp16, or bf16 for bf16 models);
// the rotation runs in float32 and rounds once to E (portable.py:130-132,
// `.astype(x.dtype)`).
template <typename E>
__device__ __forceinline__ void rotate_head(const E* src, E* dst, float pos,
                                            const float* inv_freq, int half, int d,
                                            int lane) {
  // No fused multiply-add: the products are rounded before the sum, as in the
  // reference's float32 expression (device code contracts x * y - z by default,
  // into a multiply-add that may even round straight to the 16-bit result;
  // the pragma covers the expressions written here, not those inside library
  // helpers such as __fmul_rn).
#pragma clang fp contract(off)
  for (int j = lane; j < half; j += 64) {
    const float x1 = (float)src[j];
    const float x2 = (float)src[j + half];
    float s, c;
    sincosf(pos * inv_freq[j], &s, &c);
    dst[j] = (E)(x1 * c - x2 * s);
    dst[j + half] = (E)(x2 * c + x1 * s);
  }
  for (int e = 2 * half + lane; e < d; e += 64) dst[e] = src[e];
}

// One wave per head: workgroup (t, y) takes heads 4y .. 4y + 3 of token t,
// query heads first, then kv heads. No LDS and no barrier: every wave
// computes the angles it uses (sincosf with full range reduction).
template <typename E>
__global__ __launch_bounds__(kAppendThreads) void rope_append_kernel(const AppendParams p) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * kHeadsPerGroup + (threadIdx.x >> 6);
  if (h >= p.hq + p.hkv) return;
  const float pos = p.half > 0 ? (float)p.positions[t] : 0.0f;
  if (h < p.hq) {
    const int64_t base = ((int64_t)t * p.hq + h) * p.d;
    rotate_head(reinterpret_cast<const E*>(p.q) + base, reinterpret_cast<E*>(p.q_out) + base,
                pos, p.inv_freq, p.half, p.d, lane);
    return;
  }
  const int64_t row = p.rows[t];
  if (row < 0 || row >= p.arena_rows) return;  // rows outside the arena are skipped
  const int kh = h - p.hq;
  const int64_t base = ((int64_t)t * p.hkv + kh) * p.d;
  rotate_head(reinterpret_cast<const E*>(p.k) + base,
              static_cast<E*>(p.k_arena) + arena_index(p, row, kh, 0), pos, p.inv_freq,
              p.half, p.d, lane);
  E* const vdst = static_cast<E*>(p.v_arena) + arena_index(p, row, kh, 0);
  const E* const vsrc = reinterpret_cast<const E*>(p.v) + base;
  for (int e = lane; e < p.d; e += 64) vdst[e] = vsrc[e];
}

constexpr int kMaxPerLane = kMaxHeadDim / 64;  // elements of a row per lane

// The rotated value of element e of a row (fp16, as rotate_head writes it),
// reading the element and its rotation partner.
__device__ __forceinline__ f16 rotated(const f16* src, int e, float pos, const float* inv_freq,
                                       int half) {
#pragma clang fp contract(off)
  if (e >= 2 * half) return src[e];
  const int j = e < half ? e : e - half;
  const float x1 = (float)src[j];
  const float x2 = (float)src[j + half];
  float s, c;
  sincosf(pos * inv_freq[j], &s, &c);
  return e < half ? (f16)(x1 * c - x2 * s) : (f16)(x2 * c + x1 * s);
}

// One row of one wave, lane-owned elements e = lane + 64 i, quantized as
// paged_kv.quantize (paged_kv.py:50-55): scale = fp16(max(absmax, 1e-4) /
// 127), q = clip(rint(x / scale), -127, 127).
__device__ __forceinline__ void quantize_row(const f16 (&x)[kMaxPerLane], int d, int lane,
                                             int8_t* dst, f16* scale_dst) {
  float top = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i)
    if (lane + 64 * i < d) top = fmaxf(top, fabsf((float)x[i]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) top = fmaxf(top, __shfl_xor(top, off));
  const f16 scale = (f16)(fmaxf(top, 1e-4f) / 127.0f);
  const float sf = (float)scale;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    if (e < d) {
      const float q = fminf(fmaxf(rintf((float)x[i] / sf), -127.0f), 127.0f);
      dst[e] = (int8_t)q;
    }
  }
  if (lane == 0) *scale_dst = scale;
}

// 8-bit K/V: as rope_append_kernel, with the rotated keys and the values
// quantized per (row, kv head) into int8 arenas and fp16 scale arenas.
__global__ __launch_bounds__(kAppendThreads) void rope_append_q8_kernel(const AppendParams p) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * kHeadsPerGroup + (threadIdx.x >> 6);
  if (h >= p.hq + p.hkv) return;
  const float pos = p.half > 0 ? (float)p.positions[t] : 0.0f;
  if (h < p.hq) {
    const int64_t base = ((int64_t)t * p.hq + h) * p.d;
    rotate_head(p.q + base, p.q_out + base, pos, p.inv_freq, p.half, p.d, lane);
    return;
  }
  const int64_t row = p.rows[t];
  if (row < 0 || row >= p.arena_rows) return;  // rows outside the arena are skipped
  const int kh = h - p.hq;
  const int64_t base = ((int64_t)t * p.hkv + kh) * p.d;
  f16 xk[kMaxPerLane], xv[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    xk[i] = e < p.d ? rotated(p.k + base, e, pos, p.inv_freq, p.half) : (f16)0.0f;
    xv[i] = e < p.d ? p.v[base + e] : (f16)0.0f;
  }
  const int64_t at = arena_index(p, row, kh, 0);
  const int64_t sat = scale_index(p, row, kh);
  quantize_row(xk, p.d, lane, static_cast<int8_t*>(p.k_arena) + at, p.k_scale + sat);
  quantize_row(xv, p.d, lane, static_cast<int8_t*>(p.v_arena) + at, p.v_scale + sat);
}

using pda_internal::fail;
using pda_internal::ok;

int rope_append(const void* q, void* q_out, const void* k, const void* v, void* k_arena,
                void* v_arena, void* k_scale, void* v_scale, bool q8, bool bf16_elems,
                const int32_t* positions, const int32_t* rows, int32_t n, int32_t q_heads,
                int32_t kv_heads, int32_t head_dim, int32_t page_size, int64_t arena_rows,
                int32_t layout, int32_t rope_dims, const float* inv_freq, void* stream) {
  if (n < 0 || head_dim <= 0 || head_dim > kMaxHeadDim)
    return fail(PDA_ERR_INVALID_ARGUMENT, "n=%d head_dim=%d (need n >= 0, 0 < head_dim <= %d)",
                n, head_dim, kMaxHeadDim);
  if (n == 0) return ok();  // nothing is read or written (buffers may be NULL)
  if (rope_dims < 0 || rope_dims > head_dim || rope_dims % 2)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "rope_dims %d must be even and within [0, head_dim %d]", rope_dims, head_dim);
  const bool rotate_q = q != nullptr || q_out != nullptr;
  if (rotate_q && (!q || !q_out || q_heads <= 0))
    return fail(PDA_ERR_INVALID_ARGUMENT, "queries need q, q_out and q_heads > 0");
  const bool append = k || v || k_arena || v_arena || rows || (q8 && (k_scale || v_scale));
  if (append) {
    if (!k || !v || !k_arena || !v_arena || !rows || kv_heads <= 0 ||
        (q8 && (!k_scale || !v_scale)))
      return fail(PDA_ERR_INVALID_ARGUMENT, "the K/V write needs k, v, both arenas%s, rows "
                  "and kv_heads > 0", q8 ? ", both scale arenas" : "");
    if (layout != PDA_LAYOUT_ROWS && layout != PDA_LAYOUT_PAGES)
      return fail(PDA_ERR_INVALID_ARGUMENT, "unknown K/V layout %d", layout);
    if (arena_rows <= 0 || (layout == PDA_LAYOUT_PAGES && (page_size <= 0 || arena_rows % page_size)))
      return fail(PDA_ERR_INVALID_ARGUMENT,
                  "arena_rows %lld must be positive (a multiple of page_size %d for page tiles)",
                  (long long)arena_rows, page_size);
  }
  if (rope_dims > 0 && (!positions || !inv_freq))
    return fail(PDA_ERR_INVALID_ARGUMENT, "rotation needs positions and inv_freq");
  const uintptr_t mis = (uintptr_t)q | (uintptr_t)q_out | (uintptr_t)k | (uintptr_t)v |
                        (q8 ? (uintptr_t)k_scale | (uintptr_t)v_scale
                            : (uintptr_t)k_arena | (uintptr_t)v_arena);
  if (mis & 1) return fail(PDA_ERR_ALIGNMENT, "fp16 buffers must be 2-byte aligned");
  if ((uintptr_t)positions & 3 || (uintptr_t)rows & 3 || (uintptr_t)inv_freq & 3)
    return fail(PDA_ERR_ALIGNMENT, "int32/float32 buffers must be 4-byte aligned");
  const int hq = rotate_q ? q_heads : 0;
  const int hkv = append ? kv_heads : 0;
  if (hq + hkv == 0) return ok();
  if ((int64_t)hq + hkv > 65535LL * kHeadsPerGroup)
    return fail(PDA_ERR_INVALID_ARGUMENT, "too many heads (%d)", hq + hkv);

  AppendParams prm;
  prm.q = static_cast<const f16*>(q);
  prm.q_out = static_cast<f16*>(q_out);
  prm.k = static_cast<const f16*>(k);
  prm.v = static_cast<const f16*>(v);
  prm.k_arena = k_arena;
  prm.v_arena = v_arena;
  prm.k_scale = static_cast<f16*>(k_scale);
  prm.v_scale = static_cast<f16*>(v_scale);
  prm.positions = positions;
  prm.rows = rows;
  prm.inv_freq = inv_freq;
  prm.arena_rows = arena_rows;
  prm.hq = hq;
  prm.hkv = hkv;
  prm.d = head_dim;
  prm.half = rope_dims / 2;
  prm.page_size = page_size;
  prm.layout = layout;
  void* args[] = {&prm};
  const dim3 grid(n, (hq + hkv + kHeadsPerGroup - 1) / kHeadsPerGroup);
  const void* fn = q8     ? reinterpret_cast<const void*>(rope_append_q8_kernel)
                   : bf16_elems ? reinterpret_cast<const void*>(rope_append_kernel<bf16>)
                          : reinterpret_cast<const void*>(rope_append_kernel<f16>);
  const hipError_t err = hipLaunchKernel(fn, grid, dim3(kAppendThreads), args, 0,
                                         static_cast<hipStream_t>(stream));
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

}  // namespace

extern "C" {

int pda_rope_append(const void* q, void* q_out, const void* k, const void* v,
                    void* k_arena, void* v_arena, const int32_t* positions,
                    const int32_t* rows, int32_t n, int32_t q_heads, int32_t kv_heads,
                    int32_t head_dim, int32_t page_size, int64_t arena_rows,
                    int32_t layout, int32_t rope_dims, const float* inv_freq,
                    void* stream) {
  return rope_append(q, q_out, k, v, k_arena, v_arena, nullptr, nullptr, false, false,
                     positions, rows, n, q_heads, kv_heads, head_dim, page_size, arena_rows,
                     layout, rope_dims, inv_freq, stream);
}

int pda_rope_append_bf16(const void* q, void* q_out, const void* k, const void* v,
                         void* k_arena, void* v_arena, const int32_t* positions,
                         const int32_t* rows, int32_t n, int32_t q_heads, int32_t kv_heads,
                         int32_t head_dim, int32_t page_size, int64_t arena_rows,
                         int32_t layout, int32_t rope_dims, const float* inv_freq,
                         void* stream) {
  return rope_append(q, q_out, k, v, k_arena, v_arena, nullptr, nullptr, false, true,
                     positions, rows, n, q_heads, kv_heads, head_dim, page_size, arena_rows,
                     layout, rope_dims, inv_freq, stream);
}

int pda_rope_append_q8(const void* q, void* q_out, const void* k, const void* v,
                       void* k_arena, void* v_arena, void* key_scales, void* value_scales,
                       const int32_t* positions, const int32_t* rows, int32_t n,
                       int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                       int32_t page_size, int64_t arena_rows, int32_t layout,
                       int32_t rope_dims, const float* inv_freq, void* stream) {
  return rope_append(q, q_out, k, v, k_arena, v_arena, key_scales, value_scales, true, false,
                     positions, rows, n, q_heads, kv_heads, head_dim, page_size, arena_rows,
                     layout, rope_dims, inv_freq, stream);
}

}  // extern "C"
