// Split-K paged decode attention for MI355X (gfx950 / CDNA4), C-ABI in pda.h.
//
// Reference algorithm: python/instinct/backends/metal_kernels.py:18-124
// (pass one _DECODE_BODY, tails _SINGLE_WRITE/_SPLIT_WRITE, merge
// _DECODE_MERGE) and its host wrapper paged_decode_attention (:164-248).
// The semantics are those of the portable path (portable.py:155-205): visible
// keys are [max(0, len - window), len), pages with a negative id are masked.
//
// MI355X design (not a translation of the Metal kernel):
//  * Stream split. A unit is (sequence, kv head group); the visible pages of
//    all units, in order, form one stream of T pages. A persistent grid of
//    eight-wave workgroups (one per CU at two waves per SIMD) cuts the stream
//    into equal contiguous ranges, one per wave pair. The two waves of a pair
//    share a SIMD (waves i and i + 4 of a workgroup); the SIMD's issue arbiter
//    favours the older of two waves, which then streams up to ~20% faster, so
//    a fixed split would leave half the waves idle at the end. The pair
//    therefore takes its range from both ends, the first wave forward and the
//    second backward, one page per ticket of a shared LDS counter, and meets
//    wherever the tickets run out. Each wave still ends with one contiguous
//    range, cut by the meeting point instead of a fixed boundary (the
//    reference splits every sequence by the longest one,
//    metal_kernels.py:193-194).
//  * A unit that lies inside one wave's range is normalised and written by
//    that wave (as _SINGLE_WRITE); a unit cut by a range boundary leaves
//    unnormalised partials (as _SPLIT_WRITE) in one of the wave's two slots,
//    which the merge kernel combines (as _DECODE_MERGE). The first wave of
//    each pair records the meeting point for the merge. (Merging in the
//    split kernel was measured slower: agent-scope fences at every cut unit
//    write back the L2 and more than doubled the kernel on config 3, and a
//    fence-free variant, device-coherent stores plus a per-unit counter,
//    left one wave to read all pieces of a unit at the very end.)
//  * Inside a wave, R lanes share one key row (R = head_dim / EPL, EPL = 8 or
//    16 fp16 per lane, i.e. one or two 16-byte loads per lane per row), so a
//    wave covers 64 / R keys per step. Every step reads K and V rows once and
//    serves all G query heads of the GQA group from registers.
//  * q.k uses v_dot2 (fp16 pairs, fp32 accumulate) and a DPP butterfly over
//    the R lanes. p.v uses v_dot2 over key pairs where the head dim allows it
//    (128, 256, 512: fp16 probabilities of two keys times their fp16 values),
//    else mixed-precision FMA (fp32 += fp32 * fp16).
//  * Online softmax in the log2 domain with a lazy running max: the
//    accumulators are rescaled only when a score exceeds the running max by
//    more than 2^8, so steady-state steps do no rescaling.
//  * K/V loads run NBUF steps ahead of the math through a register ring, and
//    the ticket for the next page is taken one page ahead.
//  * No cross-workgroup synchronisation: the split kernel only writes, the
//    merge kernel runs after it on the same stream.

#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <stdarg.h>
#include <stdlib.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <utility>

#include "pda.h"
#include "pda_decode.h"
#include "pda_internal.h"

namespace pda_internal {

namespace {
thread_local char g_error[512] = "";
}  // namespace

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

const char* last_error() { return g_error; }

}  // namespace pda_internal

namespace {

using namespace pda_decode;
using pda_internal::fail;
using pda_internal::ok;

// Head dims with a compiled fast path: 16-bit 64, 80, 96, 128, 256, 512;
// 8-bit 64, 128, 256, 512 (the dims whose p.v runs on key pairs). Every
// other head dim up to 512 runs a generic kernel padded to a power of two
// (any dim at 8 bits that has no fast path, 80 included; odd ones the odd
// variant, one query head per unit).
bool fast_dim(int d, bool q8) {
  if (q8) return d == 64 || d == 128 || d == 256 || d == 512;
  return d == 64 || d == 80 || d == 96 || d == 128 || d == 256 || d == 512;
}

// Padded head dim of a generic kernel: the next power of two, at least 8.
int generic_dim(int d) {
  int dp = 8;
  while (dp < d) dp <<= 1;
  return dp;
}

// The head dim the kernels lay partials out on: d, or its generic padding.
int kernel_dim(int d, bool q8) { return fast_dim(d, q8) ? d : generic_dim(d); }

// Partial row length the workspace is sized for: the larger of the 16-bit
// and 8-bit layouts, so pda_workspace_bytes holds for either cache.
int workspace_dim(int d) { return std::max(kernel_dim(d, false), kernel_dim(d, true)); }

KernelPair kernels_for(int d, int g, bool q8, bool bf16 = false) {
  if (d <= 0 || d > 512) return {};
  if (d % 2) return g == 1 ? kernels_odd(generic_dim(d), q8, bf16) : KernelPair{};
  if (fast_dim(d, q8)) {
    if (q8) return bf16 ? kernels_q8_bf16(d, g) : kernels_q8(d, g);
    return bf16 ? kernels_bf16(d, g) : kernels_f16(d, g);
  }
  const int dp = generic_dim(d);
  if (q8) return bf16 ? kernels_gen_q8_bf16(dp, g) : kernels_gen_q8(dp, g);
  return bf16 ? kernels_gen_bf16(dp, g) : kernels_gen_f16(dp, g);
}

// Keys one wave step covers for a head dim (generic kernels: 8 elements per
// lane, so 64 / (dp / 8) keys).
int keys_per_step(int d, bool q8) {
  if (!fast_dim(d, q8)) return 64 / (generic_dim(d) / 8);
  if (q8) {
    switch (d) {
      case 64: return Geom<64, true>::KPS;
      case 128: return Geom<128, true>::KPS;
      case 256: return Geom<256, true>::KPS;
      case 512: return Geom<512, true>::KPS;
    }
    return 0;
  }
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

// Heads per unit on the VALU kernels: the whole GQA group when it has at
// most 8 heads, otherwise the largest divisor of it that does.
int heads_per_group(int gtot) {
  for (int g = gtot < 8 ? gtot : 8; g >= 1; --g)
    if (gtot % g == 0) return g;
  return 1;
}

// Matrix-core kernels: head dims whose rows split into 32-element chunks
// (64-element ones at 8 bits), and GQA groups of at least mf_min_group(q8, d)
// heads (the PDA_MFMA_MIN_GROUP environment variable moves both thresholds,
// for measurements). 16-bit K/V: from 5 heads on, the VALU's q.k and p.v
// issue of the 8-wave workgroup costs more than the matrix cores' 16-head
// tiles with idle head slots (config 2's lengths, D 64 to 256); at 4 heads
// and fewer the VALU kernels are faster. 8-bit K/V: the VALU kernels spend
// most of their issue on the int8 conversions, which the matrix-core kernel
// does once per element for all heads; it is level or faster at every group
// size measured (1 to 7 heads, configs 1-5: config 2 114.7 -> 74.1 us).
// D = 512 (four-wave workgroups, one K/V step in flight per wave), on the
// Gemma 4 global layer (2 kv heads, 261,840 tokens): at 16 bits the
// matrix-core kernel is faster at every group (191-196 us against the VALU
// kernel's 197-222 at 1-8 heads); at 8 bits it takes 131-135 us at any
// group, the VALU kernel 117-131 us at 1-3 heads and 157-217 at 4-8, so
// 8-bit D = 512 starts at 4 heads.
bool mf_dim(int d, bool q8) {
  return q8 ? (d == 64 || d == 128 || d == 256 || d == 512)
            : (d == 64 || d == 96 || d == 128 || d == 256 || d == 512);
}

int mf_min_group(bool q8, int d) {
  static const int env = [] {
    const char* e = getenv("PDA_MFMA_MIN_GROUP");
    return e ? atoi(e) : 0;
  }();
  if (env > 0) return env;
  if (d == 512) return q8 ? 4 : 1;
  return q8 ? 1 : 5;
}

bool use_mf(int gtot, int d, bool q8) { return mf_dim(d, q8) && gtot >= mf_min_group(q8, d); }

// Heads per unit on the matrix cores: the whole group when it has at most 16
// heads (one K/V read serves them all), else the largest divisor that does.
int mf_unit_heads(int gtot) {
  for (int g = gtot < 16 ? gtot : 16; g >= 1; --g)
    if (gtot % g == 0) return g;
  return 1;
}

struct Plan {
  int G = 0;           // partial slots per unit (the kernels' head slots)
  int unit_heads = 0;  // query heads of a unit
  int nhg = 0;         // units per kv head
  bool mf = false;     // matrix-core kernels
  int min_pages = 0;
  int64_t pages_est = 0;       // visible pages of the batch if every length = longest
  int64_t unit_pages_max = 0;  // visible pages of one unit, at most
  size_t off_meet = 0, off_ml = 0, off_o = 0, total = 0;
};


size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int make_plan(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
              int32_t page_size, int32_t table_stride, int32_t longest,
              int32_t window, int32_t split_pages, Plan* out, bool q8 = false) {
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      page_size <= 0 || table_stride <= 0 || window < 0 || split_pages < 0)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "non-positive size (batch=%d q_heads=%d kv_heads=%d head_dim=%d "
                "page_size=%d table_stride=%d window=%d split_pages=%d)",
                batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                window, split_pages);
  if (q_heads % kv_heads)
    return fail(PDA_ERR_HEAD_RATIO, "query heads must be a multiple of kv heads");
  if (head_dim > 512)
    return fail(PDA_ERR_HEAD_DIM, "head_dim %d is above 512", head_dim);
  if ((int64_t)table_stride * page_size > INT32_MAX)
    return fail(PDA_ERR_TOO_LONG, "table_stride * page_size exceeds 2^31");
  if (batch > kMaxBatch)
    return fail(PDA_ERR_INVALID_ARGUMENT, "batch %d above %d", batch, kMaxBatch);
  Plan pl;
  const int gtot = q_heads / kv_heads;
  pl.mf = use_mf(gtot, head_dim, q8);
  // Odd head dims: one query head per unit (the only odd instantiation).
  pl.unit_heads = head_dim % 2 ? 1 : pl.mf ? mf_unit_heads(gtot) : heads_per_group(gtot);
  pl.G = pl.mf ? 16 : pl.unit_heads;
  pl.nhg = gtot / pl.unit_heads;
  // The workspace holds the widest slot layout either cache type could use
  // for this shape (pda_workspace_bytes does not know the element type).
  const int g_ws = std::max(
      use_mf(gtot, head_dim, false) ? mf_unit_heads(gtot) : heads_per_group(gtot),
      use_mf(gtot, head_dim, true) ? mf_unit_heads(gtot) : heads_per_group(gtot));
  if ((int64_t)kv_heads * pl.nhg > 65535)
    return fail(PDA_ERR_INVALID_ARGUMENT, "kv heads x head groups above 65535");
  // Visible pages of one sequence are bounded by the table width and, with a
  // window, by the pages a window can touch.
  int64_t pages_max = table_stride;
  if (window > 0) pages_max = std::min<int64_t>(pages_max, (window - 1) / page_size + 2);
  if ((int64_t)batch * pages_max * kv_heads * pl.nhg > INT32_MAX)
    return fail(PDA_ERR_TOO_LONG, "more than 2^31 visible pages in one call");
  int64_t est = pages_max;
  if (longest > 0) est = std::min<int64_t>(est, (longest + page_size - 1) / page_size + 1);
  pl.unit_pages_max = est;
  pl.pages_est = (int64_t)batch * kv_heads * pl.nhg * est;
  pl.min_pages = split_pages > 0 ? split_pages : kMinPagesPerWave;
  // Workspace: the per-sequence page prefix, the meeting points of the wave
  // pairs, the (max, sum) pairs and the unnormalised partial outputs of the
  // cut units (two slots per wave). Nothing in it outlives a call, so calls
  // of any shape share one workspace without initialisation.
  pl.off_meet = align256((size_t)(batch + 1) * sizeof(int32_t));
  pl.off_ml = pl.off_meet + align256((size_t)kMaxPairs * sizeof(int32_t));
  pl.off_o = pl.off_ml + align256((size_t)kSlots * g_ws * sizeof(float2));
  pl.total = pl.off_o + align256((size_t)kSlots * g_ws * workspace_dim(head_dim) * sizeof(float));
  *out = pl;
  return PDA_OK;
}

// Resident workgroups of a split kernel on the current device (cached).
int resident_groups(KernelFn fn, int threads, size_t lds_bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, std::pair<const void*, size_t>>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  const auto key = std::make_pair(dev, std::make_pair((const void*)fn, lds_bytes));
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                   threads, lds_bytes) != hipSuccess)
    return -1;
  const int groups = std::max(1, std::min(kMaxGroups, cus * std::max(1, per_cu)));
  cache[key] = groups;
  return groups;
}

// Merge launch. Units with many pieces (a few long sequences) take the
// row-sliced kernel: a workgroup per 64-element slice of a head's row and
// rounds of 64 pieces per wave, read with 16-byte loads and one (max, sum)
// load per piece; with one workgroup per head, hundreds of pieces would be
// read whole-row on a few CUs, 32 pieces or fewer per round, every lane
// loading each piece's (max, sum). Waves: enough for one round per wave on
// the longest unit (its pieces estimated from `longest`), 16 at most. `dim`
// is the kernels' head dim (the partials' row length), `heads` the merge
// workgroups before slicing.
struct MergeShape {
  bool sliced;
  int slices;  // workgroups per head
  int waves;   // per workgroup
};

MergeShape merge_shape(const Plan& pl, int dim, int grid_pairs, int64_t heads) {
  const int64_t pairs = std::max<int64_t>(
      1, std::min<int64_t>(grid_pairs, (pl.pages_est + 2 * pl.min_pages - 1) /
                                           (2 * pl.min_pages)));
  const int64_t per_pair = std::max<int64_t>(1, pl.pages_est / pairs);
  const int64_t pieces = 2 * (pl.unit_pages_max / per_pair + 2);
  const int chunks = (dim + 63) / 64;
  // PDA_MERGE_SLICED=0/1 forces the choice (for measurements); results
  // differ only in summation order.
  static const int force = [] {
    const char* e = getenv("PDA_MERGE_SLICED");
    return e && *e ? atoi(e) : -1;
  }();
  const bool sliced = force >= 0 ? force > 0
                                 : pieces > kMergeSlicedRound &&
                                       heads * chunks <= kMergeSlicedMaxGroups;
  const int per_round = sliced ? kMergeSlicedRound : 32 / chunks;
  const int64_t mw = (pieces + per_round - 1) / per_round;
  return {sliced, sliced ? chunks : 1,
          (int)std::max<int64_t>(1, std::min<int64_t>(kMergeMaxWaves, mw))};
}

// Local mode: one split workgroup per unit, its waves' pieces merged in
// LDS at the end, no merge pass. It saves the merge's launch, its gap
// after the split kernel and its dependent loads (~6.5 us between events),
// but a unit's pages go to one workgroup's waves instead of being spread
// over the whole GPU, so it is chosen where that costs a wave few more
// pages than the stream gives it, scaled by the steps its ring keeps in
// flight (ring / 4 x 2.5 times): config 4's windows with the 4-deep VALU
// ring (128 units of ~65 pages: 8 pages a wave against 4; 39.8 -> 37.2 us),
// not at 8 bits (the 1-deep matrix-core ring: 31.6 -> 33.3 us) nor config 1
// (16 units of 65 pages: 8 against 0.5; 17.5 -> 18.1 us). At most
// kLocalMaxUnits units of at most kLocalMaxUnitBytes of K/V each (from
// `longest`), pieces within kLocalMaxLds bytes of LDS. PDA_DECODE_LOCAL=0/1
// forces the choice where the pieces fit (for measurements). Returns the
// dynamic LDS bytes of the local kernel launch, or 0 for the stream.
constexpr int64_t kLocalMaxUnits = 512;
constexpr int64_t kLocalMaxUnitBytes = int64_t(3) << 19;  // 1.5 MiB
constexpr size_t kLocalMaxLds = size_t(64) << 10;

size_t local_lds(const Plan& pl, int batch, int kv_heads, int dim, int elem, int page_size,
                 int waves, int ring, int grid_pairs) {
  const size_t lds = (size_t)pda_decode::local_lds_offset(batch) * sizeof(int32_t) +
                     (size_t)waves * pl.unit_heads * (dim * sizeof(float) + sizeof(float2));
  if (lds > kLocalMaxLds) return 0;
  static const int force = [] {
    const char* e = getenv("PDA_DECODE_LOCAL");
    return e && *e ? atoi(e) : -1;
  }();
  if (force >= 0) return force > 0 ? lds : 0;
  const int64_t units = (int64_t)batch * kv_heads * pl.nhg;
  const int64_t unit_bytes = pl.unit_pages_max * page_size * (int64_t)dim * elem * 2;
  // Pages a wave takes: unit_pages_max / waves here, pages_est / (2 pairs)
  // in the stream.
  const int64_t pairs = std::max<int64_t>(
      1, std::min<int64_t>(grid_pairs, (pl.pages_est + 2 * pl.min_pages - 1) /
                                           (2 * pl.min_pages)));
  const bool short_waves = 16 * pl.unit_pages_max * pairs <= 5 * ring * waves * pl.pages_est;
  return units <= kLocalMaxUnits && unit_bytes <= kLocalMaxUnitBytes && short_waves ? lds : 0;
}

}  // namespace

extern "C" {

int pda_version(void) { return (0 << 16) | 6; }

const char* pda_last_error(void) { return pda_internal::last_error(); }

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

int pda_plan(int32_t batch, int32_t q_heads, int32_t kv_heads,
             int32_t head_dim, int32_t page_size, int32_t table_stride,
             int32_t longest, int32_t window, int32_t split_pages,
             int32_t* waves, int32_t* pages_per_wave) {
  if (!waves || !pages_per_wave)
    return fail(PDA_ERR_INVALID_ARGUMENT, "output pointer is null");
  Plan pl;
  const int rc = make_plan(batch, q_heads, kv_heads, head_dim, page_size,
                           table_stride, longest, window, split_pages, &pl);
  if (rc) return rc;
  // On MI355X (256 CUs, one split workgroup each): 1024 pairs at most (512
  // with the four-wave workgroups of the matrix-core kernels at D = 512).
  const int64_t want = (pl.pages_est + 2 * pl.min_pages - 1) / (2 * pl.min_pages);
  const int64_t pairs = std::max<int64_t>(
      1, std::min<int64_t>(want, 256 * split_waves(pl.mf ? head_dim : 0, pl.mf) / 2));
  *waves = (int32_t)(2 * pairs);
  *pages_per_wave = (int32_t)((pl.pages_est + *waves - 1) / *waves);
  return ok();
}

}  // extern "C"

// Scratch of the no-allocation decode entry point
// (pda_paged_decode_attention_noalloc): the workspace lives in this
// file-scope device array, 32 MiB on every GPU the library runs on, held
// until the process ends. Host code never passes `scratch` itself to a
// kernel (on the host the name is a stand-in, not a device address); it
// passes the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[size_t(32) << 20];

namespace {

constexpr size_t kScratchBytes = sizeof(scratch);
constexpr int kPassSplit = 1;
constexpr int kPassMerge = 2;

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_address(void** ptr) {
  static std::mutex mu;
  static std::map<int, void*> addresses;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  std::lock_guard<std::mutex> lock(mu);
  auto it = addresses.find(dev);
  if (it == addresses.end()) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !address)
      return fail(PDA_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(err));
    it = addresses.emplace(dev, address).first;
  }
  *ptr = it->second;
  return PDA_OK;
}

// Workspace offsets of a call: the page prefix at 0, then the meeting
// points of `pairs` wave pairs, the (max, sum) pairs and the partial outputs
// of `slots` slots of G heads x `dim` floats.
struct WorkspaceLayout {
  size_t off_meet = 0, off_ml = 0, off_o = 0, total = 0;
};

WorkspaceLayout workspace_layout(int batch, int G, int dim, int64_t pairs, int64_t slots) {
  WorkspaceLayout w;
  w.off_meet = align256((size_t)(batch + 1) * sizeof(int32_t));
  w.off_ml = w.off_meet + align256((size_t)pairs * sizeof(int32_t));
  w.off_o = w.off_ml + align256((size_t)slots * G * sizeof(float2));
  w.total = w.off_o + align256((size_t)slots * G * dim * sizeof(float));
  return w;
}

// What a call launches: the kernels (the library's dispatch), the split
// grid, the local-mode choice and the merge shape. The grid comes from the
// current device's occupancy query; without a device (`need_device` false,
// pda_decode_describe) it is MI355X's: one split workgroup on each of 256
// CUs.
struct LaunchPlan {
  KernelPair kp;
  int groups = 0;          // split workgroups
  int dim = 0;             // the partials' row length
  size_t lds = 0;          // dynamic LDS of a stream-mode split launch
  size_t lds_local = 0;    // dynamic LDS of a local-mode launch, 0: stream mode
  MergeShape ms{false, 1, 1};
};

int plan_launch(Plan& pl, int32_t batch, int32_t kv_heads, int32_t head_dim,
                int32_t page_size, bool q8, bool bf16, bool need_device, LaunchPlan* out) {
  LaunchPlan lp;
  lp.kp = pl.mf ? (head_dim == 512 ? kernels_mf512(q8, bf16)
                   : q8 ? (bf16 ? kernels_mf_q8_bf16(head_dim) : kernels_mf_q8(head_dim))
                        : kernels_mf(head_dim, bf16))
                : kernels_for(head_dim, pl.G, q8, bf16);
  if (!lp.kp.split) return fail(PDA_ERR_HEAD_DIM, "head_dim %d has no kernel", head_dim);
  lp.lds = (size_t)(2 * batch + 1) * sizeof(int32_t);
  lp.groups = resident_groups(lp.kp.split, 64 * lp.kp.split_waves, lp.lds);
  if (lp.groups < 0) {
    if (need_device) return fail(PDA_ERR_HIP, "device query failed");
    lp.groups = 256;
  }
  const int grid_pairs = lp.groups * (lp.kp.split_waves / 2);
  lp.dim = pl.mf ? head_dim : kernel_dim(head_dim, q8);
  lp.lds_local = local_lds(pl, batch, kv_heads, lp.dim, q8 ? 1 : 2, page_size,
                           lp.kp.split_waves, lp.kp.ring, grid_pairs);
  // Local mode on the VALU kernels, when a unit per GQA group leaves CUs
  // idle: a unit per query head, as long as the units still fit one
  // workgroup per resident slot. The units of one kv head read the same
  // K/V; the split kernel puts them on one XCD, whose L2 serves the repeat
  // reads (config 4: 128 -> 256 workgroups, 37.1 -> 35.6 us between events,
  // bitwise the same output). PDA_LOCAL_HEAD_UNITS=0 keeps the GQA units
  // (a measurement knob).
  static const int head_units_env = [] {
    const char* e = getenv("PDA_LOCAL_HEAD_UNITS");
    return e && *e ? atoi(e) : -1;
  }();
  if (lp.lds_local > 0 && !pl.mf && pl.unit_heads > 1 && head_units_env != 0) {
    const int64_t units = (int64_t)batch * kv_heads * pl.nhg * pl.unit_heads;
    const KernelPair k1 = kernels_for(head_dim, 1, q8, bf16);
    const size_t lds1 = (size_t)pda_decode::local_lds_offset(batch) * sizeof(int32_t) +
                        (size_t)k1.split_waves * (lp.dim * sizeof(float) + sizeof(float2));
    if (k1.split && units <= lp.groups && units <= kLocalMaxUnits && lds1 <= kLocalMaxLds) {
      pl.pages_est *= pl.unit_heads;
      pl.nhg *= pl.unit_heads;
      pl.unit_heads = 1;
      pl.G = 1;
      lp.kp = k1;
      lp.lds_local = lds1;
    }
  }
  const int heads = kv_heads * pl.nhg * pl.unit_heads;
  lp.ms = merge_shape(pl, lp.dim, grid_pairs, (int64_t)heads * batch);
  *out = lp;
  return PDA_OK;
}

// Validates, plans and launches the split pass, the merge pass or both.
// key_scales / value_scales non-null: 8-bit K/V (int8 arenas); bf16: q, K/V
// and out in bf16 instead of fp16.
int decode(int passes, const void* queries, const void* keys, const void* values,
           const void* key_scales, const void* value_scales, bool bf16,
           const int32_t* tables, const int32_t* lengths, void* out, int32_t batch,
           int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size,
           int32_t table_stride, int64_t arena_rows, int32_t layout, int32_t longest,
           float scale, int32_t window, float softcap, int32_t split_pages, int32_t flags,
           void* workspace, size_t workspace_bytes, void* stream, bool use_scratch = false) {
  const bool q8 = key_scales || value_scales;
  Plan pl;
  int rc = make_plan(batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                     longest, window, split_pages, &pl, q8);
  if (rc) return rc;
  if (batch == 0) return ok();
  if (!queries || !keys || !values || !tables || !lengths || !out ||
      (q8 && (!key_scales || !value_scales)))
    return fail(PDA_ERR_INVALID_ARGUMENT, "null buffer pointer");
  if (arena_rows < page_size)
    return fail(PDA_ERR_INVALID_ARGUMENT, "arena_rows %lld holds no whole page",
                (long long)arena_rows);
  if (layout != PDA_LAYOUT_ROWS && layout != PDA_LAYOUT_PAGES)
    return fail(PDA_ERR_INVALID_ARGUMENT, "unknown K/V layout %d", layout);
  if (flags & ~(PDA_DECODE_FIXED_SPLIT | PDA_DECODE_RACING))
    return fail(PDA_ERR_INVALID_ARGUMENT, "unknown decode flags 0x%x", flags);
  if ((flags & PDA_DECODE_FIXED_SPLIT) && (flags & PDA_DECODE_RACING))
    return fail(PDA_ERR_INVALID_ARGUMENT, "PDA_DECODE_FIXED_SPLIT and PDA_DECODE_RACING together");
  const int elem = q8 ? 1 : 2;  // bytes per K/V element
  const int64_t page_bytes = (int64_t)page_size * kv_heads * head_dim * elem;
  if (page_bytes > INT32_MAX)
    return fail(PDA_ERR_TOO_LONG, "one page of the arena exceeds 2^31 bytes");
  if (!(scale == scale) || isinf(scale) || !(softcap >= 0.0f) || isinf(softcap))
    return fail(PDA_ERR_INVALID_ARGUMENT, "scale must be finite and softcap >= 0");
  const uintptr_t mis = (uintptr_t)queries | (uintptr_t)keys | (uintptr_t)values |
                        (uintptr_t)out;
  if (mis & 15)
    return fail(PDA_ERR_ALIGNMENT, "query, K/V and output buffers must be 16-byte aligned");
  if (((uintptr_t)key_scales | (uintptr_t)value_scales) & 1)
    return fail(PDA_ERR_ALIGNMENT, "fp16 scale buffers must be 2-byte aligned");
  if ((uintptr_t)tables & 3 || (uintptr_t)lengths & 3)
    return fail(PDA_ERR_ALIGNMENT, "int32 buffers must be 4-byte aligned");
  if (!use_scratch) {
    if (!workspace || workspace_bytes < pl.total)
      return fail(PDA_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given",
                  pl.total, workspace ? workspace_bytes : (size_t)0);
    if ((uintptr_t)workspace & 255)
      return fail(PDA_ERR_ALIGNMENT, "workspace must be 256-byte aligned");
  }

  LaunchPlan lp;
  rc = plan_launch(pl, batch, kv_heads, head_dim, page_size, q8, bf16, true, &lp);
  if (rc) return rc;
  const KernelPair& kp = lp.kp;
  const size_t lds = lp.lds;
  const int wg_pairs = kp.split_waves / 2;
  const int groups = lp.groups;

  // Caller's workspace: the layout pda_workspace_bytes sizes (any grid).
  // Scratch: the same layout packed for this device's grid and this call's
  // head dim, within the scratch's fixed size.
  WorkspaceLayout wl;
  wl.off_meet = pl.off_meet;
  wl.off_ml = pl.off_ml;
  wl.off_o = pl.off_o;
  wl.total = pl.total;
  if (use_scratch) {
    wl = workspace_layout(batch, pl.unit_heads, kernel_dim(head_dim, q8), (int64_t)groups * wg_pairs,
                          (int64_t)groups * 4 * wg_pairs);
    if (wl.total > kScratchBytes)
      return fail(PDA_ERR_WORKSPACE,
                  "the no-allocation call needs %zu bytes of scratch for this shape, above "
                  "its %zu-byte maximum; call pda_paged_decode_attention with a workspace",
                  wl.total, kScratchBytes);
    rc = scratch_address(&workspace);
    if (rc) return rc;
  }

  Params prm;
  prm.q = static_cast<const f16*>(queries);
  prm.k = static_cast<const f16*>(keys);
  prm.v = static_cast<const f16*>(values);
  prm.tables = tables;
  prm.lengths = lengths;
  prm.out = static_cast<f16*>(out);
  char* ws = static_cast<char*>(workspace);
  prm.prefix = reinterpret_cast<int32_t*>(ws);
  prm.meet = reinterpret_cast<int32_t*>(ws + wl.off_meet);
  prm.part_ml = reinterpret_cast<float2*>(ws + wl.off_ml);
  prm.part_o = reinterpret_cast<float*>(ws + wl.off_o);
  prm.arena_pages = arena_rows / page_size;
  prm.page_bytes = page_bytes;
  prm.kscale = static_cast<const f16*>(key_scales);
  prm.vscale = static_cast<const f16*>(value_scales);
  prm.scale_page = (int64_t)page_size * kv_heads;
  if (layout == PDA_LAYOUT_ROWS) {  // [rows, kv_heads, head_dim], scales [rows, kv_heads]
    prm.row_bytes = kv_heads * head_dim * elem;
    prm.head_bytes = head_dim * elem;
    prm.scale_row = kv_heads;
    prm.scale_head = 1;
  } else {  // [pages, kv_heads, page_size, head_dim], scales [pages, kv_heads, page_size]
    prm.row_bytes = head_dim * elem;
    prm.head_bytes = page_size * head_dim * elem;
    prm.scale_row = 1;
    prm.scale_head = page_size;
  }
  prm.batch = batch;
  prm.table_stride = table_stride;
  prm.page_size = page_size;
  prm.hq = q_heads;
  prm.hkv = kv_heads;
  prm.head_dim = head_dim;
  prm.gtot = q_heads / kv_heads;
  prm.nhg = pl.nhg;
  prm.unit_heads = pl.unit_heads;
  prm.window = window;
  prm.grid_pairs = groups * wg_pairs;
  prm.min_pages = pl.min_pages;
  prm.fixed = (flags & PDA_DECODE_RACING) ? 0 : 1;
  // Fixed split points: how a pair's range is cut between its two waves,
  // and whether the wave that falls behind raises its issue priority. The
  // SIMD's arbiter favours the older (first) wave of a pair; racing pairs
  // meet at ~2/3 of the range on config 2's 16-bit matrix-core kernel and at
  // ~55% on the 8-bit kernels (configs 2 and 5). 16-bit: equal halves with
  // the priority steering (which keeps the pair's throughput: 112.2 vs 111.4
  // us racing on config 2). 8-bit: the steering costs a fifth of the pair's
  // throughput (the 8-bit kernel's issue mix runs slower when the priority
  // flips), so it is off and the first wave takes 142/256 of the range
  // (config 2: 87.3 -> 76.6 us, racing 75.7; config 5: 1235 -> 1055 us,
  // racing 1032). Four-wave workgroups put a pair on two SIMDs: halves.
  // PDA_FIXED_BALANCE=0/1 and PDA_FIXED_SHARE=1..255 override both
  // (measurement knobs).
  static const int balance_env = [] {
    const char* e = getenv("PDA_FIXED_BALANCE");
    return e && *e ? atoi(e) : -1;
  }();
  static const int share_env = [] {
    const char* e = getenv("PDA_FIXED_SHARE");
    return e && *e ? std::min(255, std::max(1, atoi(e))) : 0;
  }();
  const bool eight_waves = kp.split_waves == 8;
  prm.balance = balance_env >= 0 ? balance_env : (q8 ? 0 : 1);
  prm.front256 = share_env > 0 ? share_env : (q8 && eight_waves ? 142 : 128);
  const size_t lds_local = lp.lds_local;
  prm.local = lds_local > 0 ? 1 : 0;
  prm.ragged = page_size % (pl.mf ? 16 : keys_per_step(head_dim, q8)) ? 1 : 0;
  prm.scale_log2 = scale * kLog2e;
  prm.softcap = softcap;
  prm.cap_in = softcap > 0.0f ? 2.0f * kLog2e * scale / softcap : 0.0f;
  prm.cap_out = softcap * kLog2e;

  const hipStream_t st = static_cast<hipStream_t>(stream);
  void* args[] = {&prm};
  hipError_t err = hipSuccess;
  if (passes & kPassSplit) {
    // Local mode: a workgroup per unit (the merge happens inside it).
    const unsigned grid = prm.local ? (unsigned)(batch * kv_heads * pl.nhg) : (unsigned)groups;
    err = hipLaunchKernel(reinterpret_cast<const void*>(kp.split), dim3(grid),
                          dim3(64 * kp.split_waves), args, prm.local ? lds_local : lds, st);
  }
  if (err == hipSuccess && (passes & kPassMerge) && !prm.local) {
    const int heads = kv_heads * pl.nhg * pl.unit_heads;
    const MergeShape& ms = lp.ms;
    err = hipLaunchKernel(reinterpret_cast<const void*>(ms.sliced ? kp.merge_sliced : kp.merge),
                          dim3(heads * ms.slices, batch), dim3(64 * ms.waves), args, 0, st);
  }
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

}  // namespace

extern "C" {

#define PDA_DECODE_PARAMS                                                      \
  const void *queries, const void *keys, const void *values,                   \
      const int32_t *tables, const int32_t *lengths, void *out, int32_t batch, \
      int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size,  \
      int32_t table_stride, int64_t arena_rows, int32_t layout,                \
      int32_t longest, float scale, int32_t window, float softcap,             \
      int32_t split_pages, int32_t flags, void *workspace,                     \
      size_t workspace_bytes, void *stream
#define PDA_DECODE_ARGS(BF16)                                                  \
  queries, keys, values, nullptr, nullptr, BF16, tables, lengths, out, batch,  \
      q_heads, kv_heads, head_dim, page_size, table_stride, arena_rows,        \
      layout, longest, scale, window, softcap, split_pages, flags, workspace,  \
      workspace_bytes, stream
#define PDA_DECODE_PARAMS_Q8                                                   \
  const void *queries, const void *keys, const void *values,                   \
      const void *key_scales, const void *value_scales,                        \
      const int32_t *tables, const int32_t *lengths, void *out, int32_t batch, \
      int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t page_size,  \
      int32_t table_stride, int64_t arena_rows, int32_t layout,                \
      int32_t longest, float scale, int32_t window, float softcap,             \
      int32_t split_pages, int32_t flags, void *workspace,                     \
      size_t workspace_bytes, void *stream
#define PDA_DECODE_ARGS_Q8(BF16)                                               \
  queries, keys, values, key_scales, value_scales, BF16, tables, lengths, out, \
      batch, q_heads, kv_heads, head_dim, page_size, table_stride, arena_rows, \
      layout, longest, scale, window, softcap, split_pages, flags, workspace,  \
      workspace_bytes, stream

int pda_decode_describe(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                        int32_t page_size, int32_t table_stride, int32_t longest,
                        int32_t window, int32_t split_pages, int32_t kv_bits, int32_t bf16,
                        pda_decode_info* info) {
  if (!info) return fail(PDA_ERR_INVALID_ARGUMENT, "info is null");
  if (kv_bits != 16 && kv_bits != 8)
    return fail(PDA_ERR_INVALID_ARGUMENT, "kv_bits must be 16 or 8, got %d", kv_bits);
  const bool q8 = kv_bits == 8;
  Plan pl;
  int rc = make_plan(batch, q_heads, kv_heads, head_dim, page_size, table_stride, longest,
                     window, split_pages, &pl, q8);
  if (rc) return rc;
  LaunchPlan lp;
  rc = plan_launch(pl, std::max(batch, 1), kv_heads, head_dim, page_size, q8, bf16 != 0, false,
                   &lp);
  if (rc) return rc;
  const KernelPair& kp = lp.kp;
  pda_decode_info d;
  memset(&d, 0, sizeof(d));
  d.kernel_dim = kp.d;
  d.head_slots = kp.g;
  d.kv_bits = kv_bits;
  d.bf16 = kp.bf;
  d.generic = kp.gen;
  d.matrix_cores = kp.mf;
  d.unit_heads = pl.unit_heads;
  d.units_per_kv_head = pl.nhg;
  d.split_waves = kp.split_waves;
  d.ring = kp.ring;
  d.grid_groups = lp.groups;
  d.local = lp.lds_local > 0;
  d.merge = d.local ? 0 : lp.ms.sliced ? 2 : 1;
  d.merge_waves = d.local ? 0 : lp.ms.waves;
  auto tf = [](bool x) { return x ? "true" : "false"; };
  if (kp.odd)
    snprintf(d.split_kernel, sizeof(d.split_kernel), "paged_decode_odd_kernel<%d,%s,%s>", kp.d,
             tf(kp.q8), tf(kp.bf));
  else
    snprintf(d.split_kernel, sizeof(d.split_kernel), "paged_decode_kernel<%d,%d,%s,%s,%s,%s>",
             kp.d, kp.g, tf(kp.q8), tf(kp.bf), tf(kp.gen), tf(kp.mf));
  if (!d.local)
    snprintf(d.merge_kernel, sizeof(d.merge_kernel), "paged_decode_merge%s_kernel<%d,%d,%s,%s>",
             lp.ms.sliced ? "_sliced" : "", kp.d, kp.g, tf(kp.bf), tf(kp.gen));
  *info = d;
  return ok();
}

int pda_paged_decode_attention(PDA_DECODE_PARAMS) {
  return decode(kPassSplit | kPassMerge, PDA_DECODE_ARGS(false));
}

int pda_decode_split(PDA_DECODE_PARAMS) { return decode(kPassSplit, PDA_DECODE_ARGS(false)); }

int pda_paged_decode_attention_noalloc(
    const void* queries, const void* keys, const void* values, const int32_t* tables,
    const int32_t* lengths, void* out, int32_t batch, int32_t q_heads, int32_t kv_heads,
    int32_t head_dim, int32_t page_size, int32_t table_stride, int64_t arena_rows,
    int32_t layout, int32_t longest, float scale, int32_t window, float softcap,
    int32_t split_pages, int32_t flags, void* stream) {
  return decode(kPassSplit | kPassMerge, queries, keys, values, nullptr, nullptr, false, tables,
                lengths, out, batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                arena_rows, layout, longest, scale, window, softcap, split_pages, flags,
                nullptr, 0, stream, true);
}

int pda_decode_merge(PDA_DECODE_PARAMS) { return decode(kPassMerge, PDA_DECODE_ARGS(false)); }

int pda_paged_decode_attention_bf16(PDA_DECODE_PARAMS) {
  return decode(kPassSplit | kPassMerge, PDA_DECODE_ARGS(true));
}

int pda_decode_split_bf16(PDA_DECODE_PARAMS) { return decode(kPassSplit, PDA_DECODE_ARGS(true)); }

int pda_decode_merge_bf16(PDA_DECODE_PARAMS) { return decode(kPassMerge, PDA_DECODE_ARGS(true)); }

int pda_paged_decode_attention_q8(PDA_DECODE_PARAMS_Q8) {
  if (!key_scales || !value_scales)
    return fail(PDA_ERR_INVALID_ARGUMENT, "8-bit K/V needs key and value scales");
  return decode(kPassSplit | kPassMerge, PDA_DECODE_ARGS_Q8(false));
}

int pda_decode_split_q8(PDA_DECODE_PARAMS_Q8) {
  if (!key_scales || !value_scales)
    return fail(PDA_ERR_INVALID_ARGUMENT, "8-bit K/V needs key and value scales");
  return decode(kPassSplit, PDA_DECODE_ARGS_Q8(false));
}

int pda_decode_merge_q8(PDA_DECODE_PARAMS_Q8) {
  if (!key_scales || !value_scales)
    return fail(PDA_ERR_INVALID_ARGUMENT, "8-bit K/V needs key and value scales");
  return decode(kPassMerge, PDA_DECODE_ARGS_Q8(false));
}

int pda_paged_decode_attention_q8_bf16(PDA_DECODE_PARAMS_Q8) {
  if (!key_scales || !value_scales)
    return fail(PDA_ERR_INVALID_ARGUMENT, "8-bit K/V needs key and value scales");
  return decode(kPassSplit | kPassMerge, PDA_DECODE_ARGS_Q8(true));
}

int pda_decode_split_q8_bf16(PDA_DECODE_PARAMS_Q8) {
  if (!key_scales || !value_scales)
    return fail(PDA_ERR_INVALID_ARGUMENT, "8-bit K/V needs key and value scales");
  return decode(kPassSplit, PDA_DECODE_ARGS_Q8(true));
}

int pda_decode_merge_q8_bf16(PDA_DECODE_PARAMS_Q8) {
  if (!key_scales || !value_scales)
    return fail(PDA_ERR_INVALID_ARGUMENT, "8-bit K/V needs key and value scales");
  return decode(kPassMerge, PDA_DECODE_ARGS_Q8(true));
}

}  // extern "C"
