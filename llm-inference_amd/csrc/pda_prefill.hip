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
//    Keys are streamed in tiles of 32 through LDS (K and V rows gathered
//    from the pages of the sequence's table, either arena layout).
//  * Each wave computes S^T = K Q^T for its 32 queries with
//    v_mfma_f32_32x32x8_f16 (D / 8 instructions per key tile). In that
//    product's accumulator layout a lane holds 16 keys of one query, which is
//    exactly the B operand layout of the next product, so the probabilities
//    P^T feed O^T += V^T P^T (D / 32 x 4 instructions) straight from
//    registers; only V^T is read from LDS.
//  * Online softmax per query in the log2 domain with a lazy running max
//    (rescale only when a score passes the max by 2^8), masks for causality,
//    the window and unusable pages, fp16 probabilities into the matrix core,
//    fp32 accumulation, normalised fp16 output.
//  * LDS rows are padded to 16 bytes past the head so the 32 lanes reading
//    one column of K hit different banks.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "pda.h"
#include "pda_internal.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kSlack = 8.0f;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQueries = 32 * kWaves;  // queries per workgroup
constexpr int kKeys = 32;              // keys per tile

struct PrefillParams {
  const f16* q;        // [count, hq, D]
  const f16* k;        // arena
  const f16* v;
  const int32_t* table;
  f16* out;            // [count, hq, D]
  int64_t arena_pages;
  int64_t page_elems;  // elements between pages of the arena
  int32_t head_elems;  // between kv heads of one page
  int32_t row_elems;   // between rows of one page and kv head
  int32_t table_len;
  int32_t start;
  int32_t count;
  int32_t hq;
  int32_t hkv;
  int32_t page_size;
  int32_t window;
  float scale_log2;
  float softcap;
  float cap_in;   // 2 log2(e) scale / softcap
  float cap_out;  // softcap log2(e)
};

template <int D>
__global__ __launch_bounds__(kThreads) void paged_prefill_kernel(const PrefillParams p) {
  constexpr int kRow = D + 8;  // LDS row (halves), 16-byte aligned
  constexpr int kChunks = D / 8;  // 16-byte pieces of a row
  __shared__ __align__(16) f16 s_k[kKeys * kRow];
  __shared__ __align__(16) f16 s_v[kKeys * kRow];
  __shared__ int s_ok[kKeys];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int n = lane & 31;   // query column of this lane
  const int hh = lane >> 5;  // which half of the key rows this lane holds
  const int h = blockIdx.y;
  const int kvh = h / (p.hq / p.hkv);
  // The last query tiles read the most keys (causal): they start first.
  const int q0 = (gridDim.x - 1 - blockIdx.x) * kQueries;
  const int q1 = min(q0 + kQueries, p.count);
  const int qi = q0 + 32 * w + n;  // this lane's query (may be past count)
  const bool q_live = qi < p.count;
  const int qpos = p.start + qi;

  // Query fragments (B operand of S^T = K Q^T): elements 8c + 4hh .. + 3.
  f16x4 qf[kChunks];
  {
    const f16* qp = p.q + ((int64_t)(q_live ? qi : 0) * p.hq + h) * D + 4 * hh;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      f16x4 x = *reinterpret_cast<const f16x4*>(qp + 8 * c);
      qf[c] = q_live ? x : f16x4{};
    }
  }

  f32x16 o[D / 32];
#pragma unroll
  for (int b = 0; b < D / 32; ++b) o[b] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  // Keys this workgroup needs: from the first visible key of its first query
  // to its last query.
  const int last = p.start + q1 - 1;
  int kmin = 0;
  if (p.window > 0) kmin = max(0, p.start + q0 - p.window + 1);

  for (int k0 = kmin; k0 <= last; k0 += kKeys) {
    // Gather the tile's K and V rows into LDS (zeros for unusable keys).
    for (int c = tid; c < kKeys * kChunks; c += kThreads) {
      const int key = c / kChunks, part = c - key * kChunks;
      const int kp = k0 + key;
      bool ok = kp <= last;
      int64_t at = 0;
      if (ok) {
        const int pi = kp / p.page_size;
        const int page = pi < p.table_len ? p.table[pi] : -1;
        ok = page >= 0 && page < p.arena_pages;
        at = (int64_t)(ok ? page : 0) * p.page_elems + (int64_t)kvh * p.head_elems +
             (int64_t)(kp - pi * p.page_size) * p.row_elems + part * 8;
      }
      f16x8 kx = f16x8{}, vx = f16x8{};
      if (ok) {
        kx = *reinterpret_cast<const f16x8*>(p.k + at);
        vx = *reinterpret_cast<const f16x8*>(p.v + at);
      }
      *reinterpret_cast<f16x8*>(s_k + key * kRow + part * 8) = kx;
      *reinterpret_cast<f16x8*>(s_v + key * kRow + part * 8) = vx;
      if (part == 0) s_ok[key] = ok;
    }
    __syncthreads();

    // S^T (32 keys x 32 queries): lane holds keys 8 (v / 4) + 4 hh + v % 4.
    f32x16 s = f32x16{};
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const f16x4 a = *reinterpret_cast<const f16x4*>(s_k + n * kRow + 8 * c + 4 * hh);
      s = __builtin_amdgcn_mfma_f32_32x32x8f16(a, qf[c], s, 0, 0, 0);
    }
    // Scores in log2 units, masked.
    float x[16];
    float top = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = 8 * (v / 4) + 4 * hh + (v % 4);
      const int kp = k0 + key;
      float t;
      if (p.softcap > 0.0f) {
        const float e = __builtin_amdgcn_exp2f(s[v] * p.cap_in);
        t = (1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f)) * p.cap_out;
      } else {
        t = s[v] * p.scale_log2;
      }
      const bool vis = q_live && s_ok[key] && kp <= qpos &&
                       (p.window <= 0 || kp > qpos - p.window);
      x[v] = vis ? t : -INFINITY;
      top = fmaxf(top, x[v]);
    }
    top = fmaxf(top, __shfl_xor(top, 32));  // the other half of this query's keys
    // Lazy running max: rescale only when a score passes it by 2^8.
    if (top > m + kSlack) {
      const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - top);
      m = top;
      l *= f;
#pragma unroll
      for (int b = 0; b < D / 32; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[b][v] *= f;
    }
    // Probabilities as the B operand of O^T += V^T P^T (keys 8j + 4hh + t).
    f16x4 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // Masked keys weigh 0 (also while this query's max is still -inf).
        const float xv = x[4 * j + t];
        const float pr = xv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(xv - m);
        const f16 ph = (f16)pr;
        l += (float)ph;
        pf[j][t] = ph;
      }
    }
#pragma unroll
    for (int b = 0; b < D / 32; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f16x4 a;
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t] = s_v[(8 * j + 4 * hh + t) * kRow + 32 * b + n];
        o[b] = __builtin_amdgcn_mfma_f32_32x32x8f16(a, pf[j], o[b], 0, 0, 0);
      }
    }
    __syncthreads();  // the next tile overwrites LDS
  }

  if (!q_live) return;
  l += __shfl_xor(l, 32);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  f16* dst = p.out + ((int64_t)qi * p.hq + h) * D;
  // O^T rows: element 32 b + 8 (v / 4) + 4 hh + v % 4 of query n.
#pragma unroll
  for (int b = 0; b < D / 32; ++b) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f16x4 y;
#pragma unroll
      for (int t = 0; t < 4; ++t) y[t] = (f16)(o[b][4 * g + t] * inv);
      *reinterpret_cast<f16x4*>(dst + 32 * b + 8 * g + 4 * hh) = y;
    }
  }
}

using pda_internal::fail;
using pda_internal::ok;

}  // namespace

extern "C" {

int pda_paged_prefill_attention(const void* queries, const void* keys, const void* values,
                                const int32_t* table, int32_t table_len, int32_t start,
                                int32_t count, void* out, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, int32_t page_size, int64_t arena_rows,
                                int32_t layout, float scale, int32_t window, float softcap,
                                void* stream) {
  if (count < 0 || start < 0 || q_heads <= 0 || kv_heads <= 0 || page_size <= 0 ||
      table_len < 0 || window < 0)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "count=%d start=%d q_heads=%d kv_heads=%d page_size=%d table_len=%d window=%d",
                count, start, q_heads, kv_heads, page_size, table_len, window);
  if (q_heads % kv_heads)
    return fail(PDA_ERR_HEAD_RATIO, "query heads must be a multiple of kv heads");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(PDA_ERR_HEAD_DIM, "head_dim %d has no prefill kernel (64, 128, 256)",
                head_dim);
  if (count == 0) return ok();
  if ((int64_t)start + count > INT32_MAX)
    return fail(PDA_ERR_TOO_LONG, "start + count exceeds 2^31");
  if (!queries || !keys || !values || !table || !out)
    return fail(PDA_ERR_INVALID_ARGUMENT, "null buffer pointer");
  if (layout != PDA_LAYOUT_ROWS && layout != PDA_LAYOUT_PAGES)
    return fail(PDA_ERR_INVALID_ARGUMENT, "unknown K/V layout %d", layout);
  if (arena_rows < page_size)
    return fail(PDA_ERR_INVALID_ARGUMENT, "arena_rows %lld holds no whole page",
                (long long)arena_rows);
  if (!(scale == scale) || isinf(scale) || !(softcap >= 0.0f) || isinf(softcap))
    return fail(PDA_ERR_INVALID_ARGUMENT, "scale must be finite and softcap >= 0");
  const uintptr_t mis = (uintptr_t)queries | (uintptr_t)keys | (uintptr_t)values |
                        (uintptr_t)out;
  if (mis & 15)
    return fail(PDA_ERR_ALIGNMENT, "fp16 buffers must be 16-byte aligned");
  if ((uintptr_t)table & 3) return fail(PDA_ERR_ALIGNMENT, "the table must be 4-byte aligned");
  if ((int64_t)q_heads > 65535)
    return fail(PDA_ERR_INVALID_ARGUMENT, "more than 65535 query heads");

  PrefillParams prm;
  prm.q = static_cast<const f16*>(queries);
  prm.k = static_cast<const f16*>(keys);
  prm.v = static_cast<const f16*>(values);
  prm.table = table;
  prm.out = static_cast<f16*>(out);
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
  prm.hq = q_heads;
  prm.hkv = kv_heads;
  prm.page_size = page_size;
  prm.window = window;
  prm.scale_log2 = scale * kLog2e;
  prm.softcap = softcap;
  prm.cap_in = softcap > 0.0f ? 2.0f * kLog2e * scale / softcap : 0.0f;
  prm.cap_out = softcap * kLog2e;
  void* args[] = {&prm};
  const void* fn = head_dim == 64    ? reinterpret_cast<const void*>(paged_prefill_kernel<64>)
                   : head_dim == 128 ? reinterpret_cast<const void*>(paged_prefill_kernel<128>)
                                     : reinterpret_cast<const void*>(paged_prefill_kernel<256>);
  const dim3 grid((count + kQueries - 1) / kQueries, q_heads);
  const hipError_t err =
      hipLaunchKernel(fn, grid, dim3(kThreads), args, 0, static_cast<hipStream_t>(stream));
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

}  // extern "C"
