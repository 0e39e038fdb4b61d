// Split-K paged decode attention for MI355X (gfx950 / CDNA4), C-ABI in pda.h.
//
// Reference algorithm: python/instinct/backends/metal_kernels.py:18-124
// (pass one _DECODE_BODY, tails _SINGLE_WRITE/_SPLIT_WRITE, merge
// _DECODE_MERGE) and its host wrapper paged_decode_attention (:164-248).
// The semantics are those of the portable path (portable.py:155-205): visible
// keys are [max(0, len - window), len), pages with a negative id are masked.
//
// MI355X design (not a translation of the Metal kernel):
//  * One workgroup = 4 wave64s = one (sequence, kv head, split). A split is a
//    fixed run of `split_pages` pages of that sequence, so each sequence gets
//    its own split count ceil(pages / split_pages) instead of the reference's
//    batch-wide count taken from the longest sequence (:193-194). Workgroups
//    beyond a sequence's split count exit at once.
//  * Inside a wave, R lanes share one key row (R = head_dim / EPL, EPL = 8 or
//    16 fp16 per lane, i.e. one or two 16-byte loads per lane per row), so a
//    wave covers 64 / R keys per step. Every step reads K and V rows once and
//    serves all G query heads of the GQA group from registers.
//  * q.k uses v_dot2 (fp16 pairs, fp32 accumulate) and a DPP butterfly over
//    the R lanes; p.v uses mixed-precision FMA (fp32 += fp32 * fp16).
//  * Online softmax in the log2 domain with a lazy running max: the
//    accumulators are rescaled only when a score exceeds the running max by
//    more than 2^8, so steady-state steps do no rescaling.
//  * K/V loads run NBUF steps ahead of the math through a register ring.
//  * The last workgroup of a sequence's splits to finish merges the partials
//    (log-sum-exp, as _DECODE_MERGE) behind an agent-scope release/acquire
//    counter, so a call is one kernel launch. Sequences with one split
//    normalise and write their output directly (as _SINGLE_WRITE).

#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "pda.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.44269504088896340736f;
// Lazy rescale threshold (log2 units): probabilities stay below 2^8.
constexpr float kSlack = 8.0f;
constexpr int kWaves = 4;            // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSplitPages = 64;   // table entries of a split live in one VGPR
constexpr int kMaxSplits = 4096;
// Split counters: one uint32 per (sequence, kv head, head group), in a
// fixed header at the start of every workspace.
constexpr int kMaxUnits = 65536;
constexpr size_t kCounterBytes = kMaxUnits * sizeof(uint32_t);
constexpr int kNbuf = 2;             // K/V steps in flight per wave
// The planner sizes splits for this many compute units (MI355X: 256), so the
// workspace size is a pure function of the shape.
constexpr int kPlanCUs = 256;

struct Params {
  const f16* q;
  const f16* k;
  const f16* v;
  const int32_t* tables;
  const int32_t* lengths;
  f16* out;
  float* part_o;      // [B * HKV * NHG][max_splits][G][D]
  float2* part_ml;    // [B * HKV * NHG][max_splits][G] (running max, sum)
  uint32_t* counters; // [B * HKV * NHG]
  int64_t arena_pages;
  int32_t table_stride;
  int32_t page_size;
  int32_t hq;
  int32_t hkv;
  int32_t gtot;       // query heads per kv head
  int32_t nhg;        // head groups per kv head (gtot / G)
  int32_t window;
  int32_t split_pages;
  int32_t max_splits;
  float scale_log2;   // scale * log2(e)
  float scale;
  float softcap;
};

constexpr int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

template <int D>
struct Geom {
  static constexpr int EPL = (D >= 80 && D % 16 == 0) ? 16 : 8;  // fp16 per lane
  static constexpr int NV = EPL / 8;                              // 16-byte loads
  static constexpr int SLICES = D / EPL;
  static constexpr int R = next_pow2(SLICES);                     // lanes per key
  static constexpr int KPS = 64 / R;                              // keys per step
  static_assert(D % EPL == 0, "head_dim must be a multiple of 8");
  static_assert(R <= 32, "head_dim too large");
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
  return x;
}

// Sum over the 64 / R key subsets (lanes r, r + R, r + 2R, ...).
template <int R>
__device__ __forceinline__ float subset_sum(float x) {
  if constexpr (R <= 4) x += __shfl_xor(x, 4);
  if constexpr (R <= 8) x += dpp<0x128>(x);  // row_ror:8 == lane ^ 8
  if constexpr (R <= 16) x += __shfl_xor(x, 16);
  if constexpr (R <= 32) x += __shfl_xor(x, 32);
  return x;
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

__device__ __forceinline__ f16x8 load16(const f16* p) {
  return *reinterpret_cast<const f16x8*>(p);
}

__device__ __forceinline__ f16x8 zero_unless(f16x8 x, bool keep) {
  i32x4 bits = __builtin_bit_cast(i32x4, x);
  bits.x = keep ? bits.x : 0;
  bits.y = keep ? bits.y : 0;
  bits.z = keep ? bits.z : 0;
  bits.w = keep ? bits.w : 0;
  return __builtin_bit_cast(f16x8, bits);
}

// One workgroup: (split, kv head group, sequence) = (blockIdx.x, .y, .z).
template <int D, int G>
__global__ __launch_bounds__(kThreads) void paged_decode_kernel(const Params p) {
  using Gm = Geom<D>;
  constexpr int EPL = Gm::EPL, NV = Gm::NV, R = Gm::R, KPS = Gm::KPS;

  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];
  __shared__ float s_M[G];
  __shared__ float s_L[G];
  __shared__ float s_o[G * D];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int kk = lane / R;  // key of the step this lane works on
  const int r = lane % R;   // slice of the head this lane holds
  const bool active = r < Gm::SLICES;
  const int d0 = active ? r * EPL : 0;

  const int split = blockIdx.x;
  const int kvg = blockIdx.y;
  const int b = blockIdx.z;
  const int kvh = kvg / p.nhg;
  const int hg = kvg - kvh * p.nhg;
  const int P = p.page_size;

  // Geometry of this sequence (metal_kernels.py:32-36), page-aligned splits.
  int len = p.lengths[b];
  len = min(max(len, 0), p.table_stride * P);
  const int first = p.window > 0 ? max(0, len - p.window) : 0;
  const int first_page = first / P;
  const int npages = len > first ? (len - 1) / P - first_page + 1 : 0;
  const int nsplit =
      max(1, min((npages + p.split_pages - 1) / p.split_pages, p.max_splits));
  if (split >= nsplit) return;
  const int split_first = first_page + split * p.split_pages;
  const int split_npages = max(0, min(p.split_pages, npages - split * p.split_pages));
  const int wave_npages =
      split_npages > w ? (split_npages - w + kWaves - 1) / kWaves : 0;
  const int spp = P / KPS;  // steps per page
  const int nsteps = wave_npages * spp;

  // Lane i holds the physical id of split page i.
  int tbl = -1;
  if (lane < split_npages)
    tbl = p.tables[(int64_t)b * p.table_stride + split_first + lane];

  // Queries of the G heads, this lane's slice, as fp16 pairs for v_dot2.
  const int h0 = kvh * p.gtot + hg * G;
  f16x2 q[G][EPL / 2];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const f16* qp = p.q + ((int64_t)b * p.hq + h0 + g) * D + d0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      f16x8 x = zero_unless(load16(qp + 8 * v), active);
#pragma unroll
      for (int i = 0; i < 4; ++i) q[g][4 * v + i] = f16x2{x[2 * i], x[2 * i + 1]};
    }
  }

  float o[G][EPL];
  float l[G];
  float m[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = 0.0f;
    m[g] = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[g][i] = 0.0f;
  }

  const int64_t row_stride = (int64_t)p.hkv * D;  // elements between arena rows
  const f16* kbase = p.k + (int64_t)kvh * D + d0 + kk * row_stride;
  const f16* vbase = p.v + (int64_t)kvh * D + d0 + kk * row_stride;

  f16x8 kb[kNbuf][NV], vb[kNbuf][NV];
  int ld_pl = 0, ld_sub = 0;  // next step to load: (wave page, step in page)
  int cp_pl = 0, cp_sub = 0;  // next step to compute

  auto load_step = [&](f16x8(&kd)[NV], f16x8(&vd)[NV]) {
    int pid = __builtin_amdgcn_readlane(tbl, w + ld_pl * kWaves);
    pid = (pid >= 0 && pid < p.arena_pages) ? pid : 0;
    const int64_t off = ((int64_t)pid * P + ld_sub * KPS) * row_stride;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      kd[v] = load16(kbase + off + 8 * v);
      vd[v] = load16(vbase + off + 8 * v);
    }
    // Advance, staying on the last step once there (the ring keeps loading
    // it; those reloads hit the cache and their data is never used).
    if (ld_pl * spp + ld_sub + 1 < nsteps) {
      if (++ld_sub == spp) {
        ld_sub = 0;
        ++ld_pl;
      }
    }
  };

  auto compute_step = [&](f16x8(&kd)[NV], f16x8(&vd)[NV]) {
    const int pidx = w + cp_pl * kWaves;
    const int pid = __builtin_amdgcn_readlane(tbl, pidx);
    const int t0 = (split_first + pidx) * P + cp_sub * KPS;
    if (++cp_sub == spp) {
      cp_sub = 0;
      ++cp_pl;
    }
    if (pid < 0 || pid >= p.arena_pages) return;  // released page: masked
    const int t = t0 + kk;
    const bool valid = t >= first && t < len;
    if (!(t0 >= first && t0 + KPS <= len)) {
      // Boundary step. A step with no visible key is skipped: before the
      // first visible key the running max is still -inf, and -inf - -inf
      // would poison the sums. Rows outside [first, len) may hold anything,
      // so their values are zeroed.
      if (!__any(valid)) return;
#pragma unroll
      for (int v = 0; v < NV; ++v) vd[v] = zero_unless(vd[v], valid);
    }
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = 0.0f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f16x2 kp = f16x2{kd[v][2 * i], kd[v][2 * i + 1]};
          acc = __builtin_amdgcn_fdot2(q[g][4 * v + i], kp, acc, false);
        }
      }
      s[g] = acc;
    }
    bool grow = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float x = group_sum<R>(s[g]);
      if (p.softcap > 0.0f) {
        x = tanhf(x * p.scale / p.softcap) * p.softcap * kLog2e;
      } else {
        x *= p.scale_log2;
      }
      x = valid ? x : -INFINITY;
      s[g] = x;
      grow |= x > m[g] + kSlack;
    }
    if (__any(grow)) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float mn = fmaxf(m[g], wave_max(s[g]));
        const float f = __builtin_amdgcn_exp2f(m[g] - mn);
        m[g] = mn;
        l[g] *= f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) o[g][i] *= f;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float pr = __builtin_amdgcn_exp2f(s[g] - m[g]);
      l[g] += pr;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          o[g][8 * v + i] = __builtin_fmaf(pr, (float)vd[v][i], o[g][8 * v + i]);
      }
    }
  };

  if (nsteps > 0) {
#pragma unroll
    for (int u = 0; u < kNbuf; ++u) load_step(kb[u], vb[u]);
    for (int j0 = 0; j0 < nsteps; j0 += kNbuf) {
#pragma unroll
      for (int u = 0; u < kNbuf; ++u) {
        if (j0 + u < nsteps) compute_step(kb[u], vb[u]);
        load_step(kb[u], vb[u]);
      }
    }
  }

  // Fold the wave's key subsets, then the waves of the workgroup
  // (metal_kernels.py:63-81, with per-wave running maxima).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = subset_sum<R>(l[g]);
#pragma unroll
    for (int i = 0; i < EPL; ++i) o[g][i] = subset_sum<R>(o[g][i]);
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_m[w][g] = m[g];
      s_l[w][g] = l[g];
    }
  }
  __syncthreads();
  if (tid < G) {
    float mx = -INFINITY;
#pragma unroll
    for (int x = 0; x < kWaves; ++x) mx = fmaxf(mx, s_m[x][tid]);
    float sum = 0.0f;
#pragma unroll
    for (int x = 0; x < kWaves; ++x)
      if (s_m[x][tid] != -INFINITY)
        sum += s_l[x][tid] * __builtin_amdgcn_exp2f(s_m[x][tid] - mx);
    s_M[tid] = mx;
    s_L[tid] = sum;
  }
  __syncthreads();
  float f[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    f[g] = m[g] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[g] - s_M[g]);
#pragma unroll
  for (int x = 0; x < kWaves; ++x) {
    if (w == x && kk == 0 && active) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          const float val = o[g][i] * f[g];
          float* dst = &s_o[g * D + d0 + i];
          *dst = x == 0 ? val : *dst + val;
        }
      }
    }
    __syncthreads();
  }

  const int nkvg = gridDim.y;
  if (nsplit == 1) {
    // Single split: normalise and write (metal_kernels.py:87-91).
    for (int idx = tid; idx < G * D; idx += kThreads) {
      const int g = idx / D;
      const int d = idx - g * D;
      const float sum = s_L[g];
      const float val = sum > 0.0f ? s_o[idx] / sum : 0.0f;
      p.out[((int64_t)b * p.hq + h0 + g) * D + d] = (f16)val;
    }
    return;
  }

  // Several splits: publish the unnormalised partial (metal_kernels.py:93-101).
  const int64_t unit = (int64_t)b * nkvg + kvg;
  const int64_t slot = unit * p.max_splits + split;
  float* po = p.part_o + slot * (G * D);
  for (int idx = tid; idx < G * D; idx += kThreads) po[idx] = s_o[idx];
  if (tid < G) p.part_ml[slot * G + tid] = make_float2(s_M[tid], s_L[tid]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(
        &p.counters[unit], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (uint32_t)(nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  // Last split to finish: log-sum-exp merge (metal_kernels.py:103-124).
  const float2* ml = p.part_ml + unit * p.max_splits * G;
  const float* ob = p.part_o + unit * p.max_splits * (G * D);
  if (w == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = -INFINITY;
      for (int s = lane; s < nsplit; s += 64) mx = fmaxf(mx, ml[s * G + g].x);
      mx = wave_max(mx);
      if (lane == 0) s_M[g] = mx;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    const float top = s_M[g];
    float acc = 0.0f, sum = 0.0f;
#pragma unroll 4
    for (int s = 0; s < nsplit; ++s) {
      const float2 e = ml[s * G + g];
      if (e.x == -INFINITY) continue;
      const float wgt = __builtin_amdgcn_exp2f(e.x - top);
      acc = __builtin_fmaf(wgt, ob[(int64_t)s * (G * D) + idx], acc);
      sum = __builtin_fmaf(wgt, e.y, sum);
    }
    const float val = sum > 0.0f ? acc / sum : 0.0f;
    p.out[((int64_t)b * p.hq + h0 + g) * D + d] = (f16)val;
  }
  if (tid == 0)
    __hip_atomic_store(&p.counters[unit], 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Host side: validation, planning, dispatch.

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_error[0] = '\0';
  return PDA_OK;
}

using KernelFn = void (*)(Params);

template <int D>
KernelFn kernel_for_g(int g) {
  switch (g) {
    case 1: return paged_decode_kernel<D, 1>;
    case 2: return paged_decode_kernel<D, 2>;
    case 3: return paged_decode_kernel<D, 3>;
    case 4: return paged_decode_kernel<D, 4>;
    case 5: return paged_decode_kernel<D, 5>;
    case 6: return paged_decode_kernel<D, 6>;
    case 7: return paged_decode_kernel<D, 7>;
    case 8: return paged_decode_kernel<D, 8>;
  }
  return nullptr;
}

KernelFn kernel_for(int d, int g) {
  switch (d) {
    case 64: return kernel_for_g<64>(g);
    case 80: return kernel_for_g<80>(g);
    case 96: return kernel_for_g<96>(g);
    case 128: return kernel_for_g<128>(g);
    case 256: return kernel_for_g<256>(g);
    case 512: return kernel_for_g<512>(g);
  }
  return nullptr;
}

int keys_per_step(int d) {
  switch (d) {
    case 64: return Geom<64>::KPS;
    case 80: return Geom<80>::KPS;
    case 96: return Geom<96>::KPS;
    case 128: return Geom<128>::KPS;
    case 256: return Geom<256>::KPS;
    case 512: return Geom<512>::KPS;
  }
  return 0;
}

// Heads per workgroup: the whole GQA group when it has at most 8 heads,
// otherwise the largest divisor of it that does.
int heads_per_group(int gtot) {
  for (int g = gtot < 8 ? gtot : 8; g >= 1; --g)
    if (gtot % g == 0) return g;
  return 1;
}

struct Plan {
  int G = 0, nhg = 0, split_pages = 0, max_splits = 0, pages_max = 0;
  size_t off_ml = 0, off_o = 0, zero_bytes = 0, total = 0;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int make_plan(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
              int32_t page_size, int32_t table_stride, int32_t longest,
              int32_t window, int32_t split_pages, Plan* out) {
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      page_size <= 0 || table_stride <= 0 || window < 0 || split_pages < 0)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "non-positive size (batch=%d q_heads=%d kv_heads=%d head_dim=%d "
                "page_size=%d table_stride=%d window=%d split_pages=%d)",
                batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                window, split_pages);
  if (q_heads % kv_heads)
    return fail(PDA_ERR_HEAD_RATIO, "query heads must be a multiple of kv heads");
  if (!kernel_for(head_dim, 1))
    return fail(PDA_ERR_HEAD_DIM,
                "head_dim %d has no kernel (supported: 64, 80, 96, 128, 256, 512)",
                head_dim);
  const int kps = keys_per_step(head_dim);
  if (page_size % kps)
    return fail(PDA_ERR_PAGE_SIZE,
                "page_size %d must be a multiple of %d for head_dim %d",
                page_size, kps, head_dim);
  if ((int64_t)table_stride * page_size > INT32_MAX)
    return fail(PDA_ERR_TOO_LONG, "table_stride * page_size exceeds 2^31");
  Plan pl;
  const int gtot = q_heads / kv_heads;
  pl.G = heads_per_group(gtot);
  pl.nhg = gtot / pl.G;
  if (batch > 65535 || (int64_t)kv_heads * pl.nhg > 65535)
    return fail(PDA_ERR_INVALID_ARGUMENT, "batch or kv head count above 65535");
  // Upper bound of visible pages of any sequence.
  int pages_max = table_stride;
  if (window > 0) pages_max = (int)std::min<int64_t>(pages_max, (window - 1) / page_size + 2);
  pl.pages_max = pages_max;
  int sp = split_pages;
  if (sp == 0) {
    int64_t est = pages_max;
    if (longest > 0) est = std::min<int64_t>(est, (longest + page_size - 1) / page_size + 1);
    const int64_t units = (int64_t)batch * kv_heads * pl.nhg;
    const int64_t target = (int64_t)kPlanCUs * 4;
    int64_t want = (units * est + target - 1) / target;
    if (want < kWaves) want = kWaves;
    if (want > kMaxSplitPages) want = kMaxSplitPages;
    sp = (int)want;
  }
  if (sp > kMaxSplitPages)
    return fail(PDA_ERR_INVALID_ARGUMENT, "split_pages %d above %d", sp, kMaxSplitPages);
  const int64_t splits = (pages_max + sp - 1) / sp;
  if (splits > kMaxSplits)
    return fail(PDA_ERR_TOO_LONG, "%lld splits of %d pages exceed %d",
                (long long)splits, sp, kMaxSplits);
  pl.split_pages = sp;
  pl.max_splits = (int)splits;
  const size_t units = (size_t)batch * kv_heads * pl.nhg;
  if (units > kMaxUnits)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "batch * kv_heads * head groups = %zu above %d", units, kMaxUnits);
  // Layout: a fixed counter header (the same for every shape, so counters
  // left at zero by one call are zero for the next call of any shape), then
  // the (max, sum) pairs and the unnormalised partial outputs.
  pl.zero_bytes = kCounterBytes;
  pl.off_ml = kCounterBytes;
  const size_t ml_bytes = align256(units * pl.max_splits * pl.G * sizeof(float2));
  pl.off_o = pl.off_ml + ml_bytes;
  const size_t o_bytes =
      align256(units * pl.max_splits * (size_t)pl.G * head_dim * sizeof(float));
  // Sequences with one split never touch the partials, but any may split.
  pl.total = pl.max_splits > 1 ? pl.off_o + o_bytes : kCounterBytes;
  *out = pl;
  return PDA_OK;
}

}  // namespace

extern "C" {

int pda_version(void) { return (0 << 16) | 1; }

const char* pda_last_error(void) { return g_error; }

int pda_workspace_bytes(int32_t batch, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, int32_t page_size,
                        int32_t table_stride, int32_t longest, int32_t window,
                        int32_t split_pages, size_t* bytes) {
  if (!bytes) return fail(PDA_ERR_INVALID_ARGUMENT, "bytes is null");
  Plan pl;
  const int rc = make_plan(batch, q_heads, kv_heads, head_dim, page_size,
                           table_stride, longest, window, split_pages, &pl);
  if (rc) return rc;
  *bytes = pl.total;
  return ok();
}

int pda_workspace_zero_bytes(size_t* bytes) {
  if (!bytes) return fail(PDA_ERR_INVALID_ARGUMENT, "bytes is null");
  *bytes = kCounterBytes;
  return ok();
}

int pda_plan(int32_t batch, int32_t q_heads, int32_t kv_heads,
             int32_t head_dim, int32_t page_size, int32_t table_stride,
             int32_t longest, int32_t window, int32_t split_pages,
             int32_t* pages_per_split, int32_t* max_splits) {
  if (!pages_per_split || !max_splits)
    return fail(PDA_ERR_INVALID_ARGUMENT, "output pointer is null");
  Plan pl;
  const int rc = make_plan(batch, q_heads, kv_heads, head_dim, page_size,
                           table_stride, longest, window, split_pages, &pl);
  if (rc) return rc;
  *pages_per_split = pl.split_pages;
  *max_splits = pl.max_splits;
  return ok();
}

int pda_paged_decode_attention(const void* queries, const void* keys,
                               const void* values, const int32_t* tables,
                               const int32_t* lengths, void* out,
                               int32_t batch, int32_t q_heads,
                               int32_t kv_heads, int32_t head_dim,
                               int32_t page_size, int32_t table_stride,
                               int64_t arena_rows, int32_t longest,
                               float scale, int32_t window, float softcap,
                               int32_t split_pages, void* workspace,
                               size_t workspace_bytes, void* stream) {
  Plan pl;
  int rc = make_plan(batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                     longest, window, split_pages, &pl);
  if (rc) return rc;
  if (batch == 0) return ok();
  if (!queries || !keys || !values || !tables || !lengths || !out)
    return fail(PDA_ERR_INVALID_ARGUMENT, "null buffer pointer");
  if (arena_rows < page_size)
    return fail(PDA_ERR_INVALID_ARGUMENT, "arena_rows %lld holds no whole page",
                (long long)arena_rows);
  if (!(scale == scale) || isinf(scale) || !(softcap >= 0.0f) || isinf(softcap))
    return fail(PDA_ERR_INVALID_ARGUMENT, "scale must be finite and softcap >= 0");
  const uintptr_t mis = (uintptr_t)queries | (uintptr_t)keys | (uintptr_t)values |
                        (uintptr_t)out;
  if (mis & 15)
    return fail(PDA_ERR_ALIGNMENT, "fp16 buffers must be 16-byte aligned");
  if ((uintptr_t)tables & 3 || (uintptr_t)lengths & 3)
    return fail(PDA_ERR_ALIGNMENT, "int32 buffers must be 4-byte aligned");
  if (!workspace || workspace_bytes < pl.total)
    return fail(PDA_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given",
                pl.total, workspace ? workspace_bytes : (size_t)0);
  if ((uintptr_t)workspace & 255)
    return fail(PDA_ERR_ALIGNMENT, "workspace must be 256-byte aligned");

  Params prm;
  prm.q = static_cast<const f16*>(queries);
  prm.k = static_cast<const f16*>(keys);
  prm.v = static_cast<const f16*>(values);
  prm.tables = tables;
  prm.lengths = lengths;
  prm.out = static_cast<f16*>(out);
  char* ws = static_cast<char*>(workspace);
  prm.counters = reinterpret_cast<uint32_t*>(ws);
  prm.part_ml = reinterpret_cast<float2*>(ws + pl.off_ml);
  prm.part_o = reinterpret_cast<float*>(ws + pl.off_o);
  prm.arena_pages = arena_rows / page_size;
  prm.table_stride = table_stride;
  prm.page_size = page_size;
  prm.hq = q_heads;
  prm.hkv = kv_heads;
  prm.gtot = q_heads / kv_heads;
  prm.nhg = pl.nhg;
  prm.window = window;
  prm.split_pages = pl.split_pages;
  prm.max_splits = pl.max_splits;
  prm.scale = scale;
  prm.scale_log2 = scale * kLog2e;
  prm.softcap = softcap;

  KernelFn fn = kernel_for(head_dim, pl.G);
  const dim3 grid(pl.max_splits, kv_heads * pl.nhg, batch);
  const dim3 block(kThreads);
  void* args[] = {&prm};
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(fn), grid, block,
                                   args, 0, static_cast<hipStream_t>(stream));
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

}  // extern "C"
