/*
 * pda.h — split-K paged decode attention for AMD Instinct MI355X (gfx950).
 *
 * C-ABI of libpda.so. Plain pointers and sizes only; every device pointer is
 * a HIP device address, `stream` is a hipStream_t (NULL = the null stream).
 * The library allocates no device memory on the call path: the caller owns
 * the queries, the K/V arenas, the page tables, the output and the workspace.
 *
 * Reference interface replaced (KavinP21/LLM-Inference, "Instinct"):
 *   paged_decode_attention(mx, queries, keys, values, tables, lengths, *,
 *                          page_size, longest, scale, window=0, softcap=0.0)
 *   python/instinct/backends/metal_kernels.py:164-248, called once per
 *   attention layer per decode step from DecodeBatch.attend
 *   (python/instinct/batches.py:203-226).
 *
 * Layouts:
 *   queries  [batch, q_heads, head_dim]            fp16
 *   keys, values: one layer's K/V arena, fp16, in one of two layouts:
 *     PDA_LAYOUT_ROWS   [arena_rows, kv_heads, head_dim] — the reference's
 *                       KVCache arena (paged_kv.py:156-292); a page is
 *                       page_size consecutive rows
 *     PDA_LAYOUT_PAGES  [arena_rows / page_size, kv_heads, page_size,
 *                       head_dim] — page tiles: the page_size rows of one
 *                       (page, kv head) are contiguous (4 KiB at head_dim 128,
 *                       page 16), so the kernel reads whole tiles; the same
 *                       logical rows, permuted within each page
 *   tables   [batch, table_stride]                 int32, physical page ids;
 *            row of logical position t = tables[b][t / page_size] * page_size
 *            + t % page_size (paged_kv.py:259-265, metal_kernels.py:47); in
 *            the page layout that row lives in tile [row / page_size][kv head],
 *            slot row % page_size
 *   lengths  [batch]                               int32, keys per sequence,
 *            the new token included (batches.py:162-164)
 *   out      [batch, q_heads, head_dim]            fp16
 *
 * Visible keys of sequence b are positions [first, lengths[b]) with
 * first = max(0, lengths[b] - window) when window > 0, else 0
 * (metal_kernels.py:32-36, portable.py:194-205). A page id that is negative
 * (a page released by the sliding-window trim, mlx_engine.py:349-372) or not
 * below arena_rows / page_size masks the keys it would hold, as the portable
 * path masks released pages (portable.py:202-204). Table entries beyond the
 * visible range are never read. A length above table_stride * page_size is
 * clamped to it; a length of zero or less yields a zero output row.
 */
#ifndef PDA_H
#define PDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. Every entry point validates its arguments on the host before
 * any HIP call and returns one of these; pda_last_error() then names the
 * problem. Mirrors the reference's ValueError for a bad head ratio
 * (metal_kernels.py:189-190). */
#define PDA_OK 0
#define PDA_ERR_INVALID_ARGUMENT (-1) /* null pointer, non-positive size, ... */
#define PDA_ERR_HEAD_RATIO (-2)       /* q_heads is not a multiple of kv_heads */
#define PDA_ERR_HEAD_DIM (-3)         /* head_dim not in 1..512               */
#define PDA_ERR_PAGE_SIZE (-4)        /* (no longer returned: any page size)  */
#define PDA_ERR_WORKSPACE (-5)        /* workspace missing or too small       */
#define PDA_ERR_ALIGNMENT (-6)        /* fp16 buffers must be 16-byte aligned */
#define PDA_ERR_TOO_LONG (-7)         /* context beyond the split planner     */
#define PDA_ERR_HIP (-8)              /* a HIP runtime call failed            */

/* Flags of the decode calls (the `flags` argument, 0 = none). */
#define PDA_DECODE_FIXED_SPLIT 1 /* fixed split points, bitwise reproducible
                                    output: the default, also taken with
                                    flags = 0 (see pda_paged_decode_attention) */
#define PDA_DECODE_RACING 2      /* opt-in: racing wave pairs, output bits may
                                    differ between calls on the same inputs */

/* K/V arena layouts (the `layout` argument of the decode calls). */
#define PDA_LAYOUT_ROWS 0  /* [rows, kv_heads, head_dim], the reference's   */
#define PDA_LAYOUT_PAGES 1 /* [pages, kv_heads, page_size, head_dim] tiles  */

/* Library version, (major << 16) | minor. No reference counterpart. */
int pda_version(void);

/* Thread-local description of the last error returned on this thread
 * ("" after success). Replaces the reference's exception text
 * (metal_kernels.py:189-190). */
const char* pda_last_error(void);

/* Bytes of device workspace pda_paged_decode_attention needs for this shape.
 * Replaces the per-call allocation of the split partials
 * (metal_kernels.py:228-239 output_shapes: partial_o [B,HQ,S,D],
 * partial_m / partial_l [B,HQ,S] in float32): here a per-sequence page
 * prefix plus two partial slots per resident wave. The workspace needs no
 * initialisation and holds nothing between calls, so one buffer serves calls
 * of any shape in turn. `longest` and `split_pages` as for the decode call. */
int pda_workspace_bytes(int32_t batch, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, int32_t page_size,
                        int32_t table_stride, int32_t longest, int32_t window,
                        int32_t split_pages, size_t* bytes);

/* The split plan for a batch whose lengths all equal `longest`: the number of
 * waves the visible pages are spread over and the pages each wave reads.
 * Informational. Replaces KEYS_PER_SPLIT / MAX_SPLITS and the batch-wide
 * split rule (metal_kernels.py:126-127,193-194): the MI355X kernel splits the
 * stream of all visible pages of the batch into equal per-wave ranges. */
int pda_plan(int32_t batch, int32_t q_heads, int32_t kv_heads,
             int32_t head_dim, int32_t page_size, int32_t table_stride,
             int32_t longest, int32_t window, int32_t split_pages,
             int32_t* waves, int32_t* pages_per_wave);

/* What a decode call of this shape launches, as the library's own dispatch
 * chooses it: for labels, profiles and measurements (no reference
 * counterpart; the reference's wrapper picks its kernels inline,
 * metal_kernels.py:193-247). The arguments are those of the decode call
 * (`kv_bits` 16 or 8, `bf16` 1 for bf16 queries and output); the split
 * grid is the current device's, or MI355X's 256 workgroups when no device is
 * visible. Local mode (`local` 1) and the merge shape depend on `batch`,
 * `longest` and the table width as the call's do. */
typedef struct pda_decode_info {
  int32_t kernel_dim;        /* D: head_dim, or the generic kernel's width     */
  int32_t head_slots;        /* G: head slots of a unit (16 on matrix cores)   */
  int32_t kv_bits;           /* 16 or 8                                        */
  int32_t bf16;              /* 1: bf16 queries, K/V and output                */
  int32_t generic;           /* 1: generic kernel (head dim without its own)   */
  int32_t matrix_cores;      /* 1: S and O products on the matrix cores        */
  int32_t unit_heads;        /* query heads one K/V read serves                */
  int32_t units_per_kv_head; /* units (head groups) per kv head                */
  int32_t split_waves;       /* waves per split workgroup                      */
  int32_t ring;              /* K/V steps in flight per wave                   */
  int32_t grid_groups;       /* split workgroups of a stream-mode launch       */
  int32_t local;             /* 1: a workgroup per unit, merged in LDS         */
  int32_t merge;             /* 0: none (local), 1: whole-row, 2: row-sliced   */
  int32_t merge_waves;       /* waves per merge workgroup                      */
  char split_kernel[96];     /* the split kernel's name and template arguments */
  char merge_kernel[96];     /* the merge kernel's ("" in local mode)          */
} pda_decode_info;

int pda_decode_describe(int32_t batch, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, int32_t page_size,
                        int32_t table_stride, int32_t longest, int32_t window,
                        int32_t split_pages, int32_t kv_bits, int32_t bf16,
                        pda_decode_info* info);

/* Paged decode attention for one new token per sequence.
 * Replaces paged_decode_attention (metal_kernels.py:164-248): same inputs and
 * meaning. `scale` multiplies q.k; `softcap` > 0 applies
 * softcap * tanh(score / softcap) (metal_kernels.py:53); `window` 0 = full
 * attention. `longest` is the host-side largest length, as in the reference
 * (a planning hint only: results never depend on it, and lengths above it
 * stay correct). `split_pages` is the fewest pages a wave reads before the
 * stream is spread over fewer waves (0 = 1; results do not depend on it
 * beyond rounding). `arena_rows` is the row count of the keys/values arenas
 * (pages x page_size) and `layout` is PDA_LAYOUT_ROWS or PDA_LAYOUT_PAGES (the
 * reference has one layout, rows); batch <= 8184. Like the reference op
 * (its IN_HEAD guard and PAGE template, metal_kernels.py:28-30,204), any
 * head_dim up to 512 and any page_size are accepted: head dims 64, 80, 96,
 * 128, 256, 512 run tuned kernels, the other even ones a generic one, odd
 * ones (rows 2-byte aligned) a generic one that moves single elements and
 * serves one query head per unit.
 * `flags`: 0 (or PDA_DECODE_FIXED_SPLIT, the same) or PDA_DECODE_RACING.
 * By default the split points are fixed by the shapes, the lengths and the
 * device's CU count, and repeated calls give bitwise-identical output, as
 * the reference's fixed split ranges do (metal_kernels.py:32-36). With
 * PDA_DECODE_RACING the two waves that share a stretch of pages split it
 * wherever their shared counter runs out (the faster wave takes more), so
 * where a sequence is cut, and the rounding of its partial results, can
 * differ between two calls on the same inputs (within the parity bar).
 * Both flags at once, or any other bit, is PDA_ERR_INVALID_ARGUMENT.
 * Launches a split kernel and a merge kernel on `stream`; calls that share a
 * workspace must not overlap. */
int pda_paged_decode_attention(const void* queries, const void* keys,
                               const void* values, const int32_t* tables,
                               const int32_t* lengths, void* out,
                               int32_t batch, int32_t q_heads,
                               int32_t kv_heads, int32_t head_dim,
                               int32_t page_size, int32_t table_stride,
                               int64_t arena_rows, int32_t layout,
                               int32_t longest, float scale, int32_t window,
                               float softcap,
                               int32_t split_pages, int32_t flags, void* workspace,
                               size_t workspace_bytes, void* stream);

/* pda_paged_decode_attention without a workspace argument: a call that
 * allocates nothing. No counterpart in the reference (its op allocates its
 * partials per call, metal_kernels.py:228-239); it is for callers that
 * cannot allocate or hand over device memory on the call path: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * The workspace is a static device array of 32 MiB per GPU inside the
 * library (held until the process ends), laid out for this device's grid;
 * a shape that needs more (about 2 x CUs x W x G x head_dim x 4 bytes, W
 * the split waves per CU: 8, or 4 for the matrix-core kernels at head_dim
 * 512; on MI355X head_dim 128 with G = 8, 256 with G = 4 and 512 with up
 * to 7 heads per kv head fit) returns PDA_ERR_WORKSPACE. Nothing in the
 * scratch outlives a call, so it needs no clearing, but every call on one
 * GPU shares it: calls that overlap on one GPU (several streams, several
 * host threads) race and must be serialised by the caller. fp16 only;
 * every other argument as for pda_paged_decode_attention. */
int pda_paged_decode_attention_noalloc(const void* queries, const void* keys,
                                       const void* values, const int32_t* tables,
                                       const int32_t* lengths, void* out,
                                       int32_t batch, int32_t q_heads,
                                       int32_t kv_heads, int32_t head_dim,
                                       int32_t page_size, int32_t table_stride,
                                       int64_t arena_rows, int32_t layout,
                                       int32_t longest, float scale,
                                       int32_t window, float softcap,
                                       int32_t split_pages, int32_t flags,
                                       void* stream);

/* The two passes of pda_paged_decode_attention, for callers that schedule or
 * time them separately; the reference's host wrapper launches the same two
 * kernels (metal_kernels.py:228-239 split, :240-247 merge). Call
 * pda_decode_split, then pda_decode_merge with the same arguments on the same
 * stream (or after it); the output is complete only after the merge. Calls
 * of few, short units run in one pass (a workgroup per unit, merged inside
 * it): their split pass writes the output and their merge pass launches
 * nothing. */
int pda_decode_split(const void* queries, const void* keys, const void* values,
                     const int32_t* tables, const int32_t* lengths, void* out,
                     int32_t batch, int32_t q_heads, int32_t kv_heads,
                     int32_t head_dim, int32_t page_size, int32_t table_stride,
                     int64_t arena_rows, int32_t layout, int32_t longest,
                     float scale, int32_t window, float softcap,
                     int32_t split_pages, int32_t flags,
                     void* workspace, size_t workspace_bytes, void* stream);
int pda_decode_merge(const void* queries, const void* keys, const void* values,
                     const int32_t* tables, const int32_t* lengths, void* out,
                     int32_t batch, int32_t q_heads, int32_t kv_heads,
                     int32_t head_dim, int32_t page_size, int32_t table_stride,
                     int64_t arena_rows, int32_t layout, int32_t longest,
                     float scale, int32_t window, float softcap,
                     int32_t split_pages, int32_t flags,
                     void* workspace, size_t workspace_bytes, void* stream);

/* bf16: the same calls with queries, K/V arenas and output in bf16, the
 * model dtype of the reference's bf16 models (their KVCache holds the model
 * dtype, paged_kv.py:156-292; the Metal kernel is templated on it,
 * metal_kernels.py:196-206). q.k and p.v run on bf16 v_dot2 (products exact,
 * fp32 accumulation); the probabilities are rounded to bf16 for p.v (and
 * the sum uses the same values). Same workspace sizing and plan. */
int pda_paged_decode_attention_bf16(const void* queries, const void* keys,
                                    const void* values, const int32_t* tables,
                                    const int32_t* lengths, void* out,
                                    int32_t batch, int32_t q_heads,
                                    int32_t kv_heads, int32_t head_dim,
                                    int32_t page_size, int32_t table_stride,
                                    int64_t arena_rows, int32_t layout,
                                    int32_t longest, float scale,
                                    int32_t window, float softcap,
                                    int32_t split_pages, int32_t flags, void* workspace,
                                    size_t workspace_bytes, void* stream);
int pda_decode_split_bf16(const void* queries, const void* keys, const void* values,
                          const int32_t* tables, const int32_t* lengths, void* out,
                          int32_t batch, int32_t q_heads, int32_t kv_heads,
                          int32_t head_dim, int32_t page_size, int32_t table_stride,
                          int64_t arena_rows, int32_t layout, int32_t longest,
                          float scale, int32_t window, float softcap,
                          int32_t split_pages, int32_t flags,
                          void* workspace, size_t workspace_bytes, void* stream);
int pda_decode_merge_bf16(const void* queries, const void* keys, const void* values,
                          const int32_t* tables, const int32_t* lengths, void* out,
                          int32_t batch, int32_t q_heads, int32_t kv_heads,
                          int32_t head_dim, int32_t page_size, int32_t table_stride,
                          int64_t arena_rows, int32_t layout, int32_t longest,
                          float scale, int32_t window, float softcap,
                          int32_t split_pages, int32_t flags,
                          void* workspace, size_t workspace_bytes, void* stream);

/* 8-bit K/V: pda_paged_decode_attention over int8 arenas with one fp16 scale
 * per (row, kv head) of keys and of values. Replaces the reference's
 * quantized path, paged_decode_attention(..., scales=(key_scales,
 * value_scales)) (metal_kernels.py:134-141,164-248 with KVCache bits=8,
 * paged_kv.py:50-55,176-181): the score is multiplied by the key's scale and
 * the probability that weights a value row by the value's scale, i.e.
 * attention over int8 * scale.
 *   keys, values  int8, [arena_rows, kv_heads, head_dim] (PDA_LAYOUT_ROWS) or
 *                 [arena_rows / page_size, kv_heads, page_size, head_dim]
 *                 (PDA_LAYOUT_PAGES), 16-byte aligned
 *   key_scales, value_scales  fp16, [arena_rows, kv_heads] beside a row
 *                 arena, [arena_rows / page_size, kv_heads, page_size] beside
 *                 a page-tile arena
 * Here K rows are converted exactly to fp16 and each score is multiplied by
 * its key's scale; V rows are dequantized to fp16(int8 x scale), the value
 * the reference's gather hands its portable path (paged_kv.py:285-292).
 * Any head_dim up to 512 (64, 128, 256 on the matrix cores at any GQA
 * group, 512 on them from 4 heads per kv head and tuned VALU kernels below,
 * the others, 80 and the odd ones included, generic); every other
 * argument as for the fp16 call, which
 * shares the workspace sizing (pda_workspace_bytes). The split and merge
 * passes exist as for fp16; merge with the _q8 entry after a _q8 split. */
int pda_paged_decode_attention_q8(const void* queries, const void* keys,
                                  const void* values, const void* key_scales,
                                  const void* value_scales,
                                  const int32_t* tables, const int32_t* lengths,
                                  void* out, int32_t batch, int32_t q_heads,
                                  int32_t kv_heads, int32_t head_dim,
                                  int32_t page_size, int32_t table_stride,
                                  int64_t arena_rows, int32_t layout,
                                  int32_t longest, float scale, int32_t window,
                                  float softcap, int32_t split_pages, int32_t flags,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);
int pda_decode_split_q8(const void* queries, const void* keys, const void* values,
                        const void* key_scales, const void* value_scales,
                        const int32_t* tables, const int32_t* lengths, void* out,
                        int32_t batch, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, int32_t page_size, int32_t table_stride,
                        int64_t arena_rows, int32_t layout, int32_t longest,
                        float scale, int32_t window, float softcap,
                        int32_t split_pages, int32_t flags, void* workspace,
                        size_t workspace_bytes, void* stream);
int pda_decode_merge_q8(const void* queries, const void* keys, const void* values,
                        const void* key_scales, const void* value_scales,
                        const int32_t* tables, const int32_t* lengths, void* out,
                        int32_t batch, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, int32_t page_size, int32_t table_stride,
                        int64_t arena_rows, int32_t layout, int32_t longest,
                        float scale, int32_t window, float softcap,
                        int32_t split_pages, int32_t flags, void* workspace,
                        size_t workspace_bytes, void* stream);

/* 8-bit K/V under a bf16 model: the _q8 calls with bf16 queries and a bf16
 * output. Replaces the reference's quantized kernel instantiated on
 * T = queries.dtype (metal_kernels.py:134-141,196-206), which a bf16 model's
 * 8-bit cache runs with bf16 queries and gets bf16 back. The int8 keys are
 * exact in fp16, so the queries are taken to fp16 scaled by a power of two
 * chosen per unit (the largest lands in [2^14, 2^15), so every bf16 value
 * converts exactly and none overflows), and each score is scaled back by the
 * same power of two; the arithmetic is then that of the _q8 calls and the
 * output is rounded once, to bf16. Arguments, workspace and passes as for
 * the _q8 calls. */
int pda_paged_decode_attention_q8_bf16(const void* queries, const void* keys,
                                       const void* values, const void* key_scales,
                                       const void* value_scales,
                                       const int32_t* tables, const int32_t* lengths,
                                       void* out, int32_t batch, int32_t q_heads,
                                       int32_t kv_heads, int32_t head_dim,
                                       int32_t page_size, int32_t table_stride,
                                       int64_t arena_rows, int32_t layout,
                                       int32_t longest, float scale, int32_t window,
                                       float softcap, int32_t split_pages, int32_t flags,
                                       void* workspace, size_t workspace_bytes,
                                       void* stream);
int pda_decode_split_q8_bf16(const void* queries, const void* keys, const void* values,
                             const void* key_scales, const void* value_scales,
                             const int32_t* tables, const int32_t* lengths, void* out,
                             int32_t batch, int32_t q_heads, int32_t kv_heads,
                             int32_t head_dim, int32_t page_size, int32_t table_stride,
                             int64_t arena_rows, int32_t layout, int32_t longest,
                             float scale, int32_t window, float softcap,
                             int32_t split_pages, int32_t flags, void* workspace,
                             size_t workspace_bytes, void* stream);
int pda_decode_merge_q8_bf16(const void* queries, const void* keys, const void* values,
                             const void* key_scales, const void* value_scales,
                             const int32_t* tables, const int32_t* lengths, void* out,
                             int32_t batch, int32_t q_heads, int32_t kv_heads,
                             int32_t head_dim, int32_t page_size, int32_t table_stride,
                             int64_t arena_rows, int32_t layout, int32_t longest,
                             float scale, int32_t window, float softcap,
                             int32_t split_pages, int32_t flags, void* workspace,
                             size_t workspace_bytes, void* stream);

/* K/V append with rotary position embedding, one launch for n tokens.
 * Replaces, per attention layer and step, the reference's
 *   q = batch.rope(q, rope_dims, ...); k = batch.rope(k, rope_dims, ...)
 *   (batches.py:195-201 -> portable.py:88-132, non-traditional RoPE) and
 *   cache.write(layer, rows, k, v) (batches.py:203-207, paged_kv.py:278-283);
 * the CUDA engine's rope_cache_kernel (cuda/kernels.cu:123-170) fuses the same.
 *   q, q_out      [n, q_heads, head_dim] fp16; q_out may equal q (in place);
 *                 both NULL: no queries
 *   k, v          [n, kv_heads, head_dim] fp16, the new keys and values
 *   k_arena, v_arena  one layer's arenas (arena_rows rows, `layout` as for the
 *                 decode call); k, v, both arenas and rows all NULL: no write
 *   positions     [n] int32, token positions (the angle offsets)
 *   rows          [n] int32, arena row of each token (table[pos / P] * P +
 *                 pos % P, batches.py:175-178); rows outside [0, arena_rows)
 *                 are not written
 *   inv_freq      [rope_dims / 2] float32 device array: angle of pair i =
 *                 float(position) * inv_freq[i] in float32, i.e.
 *                 base^(-2i / rope_dims) or 1 / freqs[i] (portable.py:117-121)
 * Element i < rope_dims / 2 of a head pairs with i + rope_dims / 2:
 *   out[i] = x[i] cos - x[i + h] sin, out[i + h] = x[i + h] cos + x[i] sin,
 * in float32, rounded to fp16; elements from rope_dims on are copied, and the
 * values are copied unchanged. rope_dims = 0 writes K/V without rotation
 * (KVCache.write alone). Requires rope_dims even, <= head_dim <= 512. No
 * workspace; enqueued on `stream`. */
int pda_rope_append(const void* q, void* q_out, const void* k, const void* v,
                    void* k_arena, void* v_arena, const int32_t* positions,
                    const int32_t* rows, int32_t n, int32_t q_heads,
                    int32_t kv_heads, int32_t head_dim, int32_t page_size,
                    int64_t arena_rows, int32_t layout, int32_t rope_dims,
                    const float* inv_freq, void* stream);

/* bf16 models: pda_rope_append with q, q_out, k, v and both arenas in bf16.
 * The rotation runs in float32 as in pda_rope_append and is rounded to bf16 to
 * nearest even, the reference's `.astype(x.dtype)` for a bf16 model
 * (portable.py:130-132); values are copied unchanged. Arguments as
 * pda_rope_append. */
int pda_rope_append_bf16(const void* q, void* q_out, const void* k, const void* v,
                         void* k_arena, void* v_arena, const int32_t* positions,
                         const int32_t* rows, int32_t n, int32_t q_heads,
                         int32_t kv_heads, int32_t head_dim, int32_t page_size,
                         int64_t arena_rows, int32_t layout, int32_t rope_dims,
                         const float* inv_freq, void* stream);

/* 8-bit K/V: pda_rope_append into int8 arenas. The rotated keys (rounded to
 * fp16 as the fp16 call writes them) and the values are quantized per (row,
 * kv head) as the reference's KVCache.write does for bits=8
 * (paged_kv.py:50-55,278-283): scale = fp16(max(absmax, 1e-4) / 127),
 * int8 = clip(rint(x / scale), -127, 127); the scales go to key_scales /
 * value_scales ([arena_rows, kv_heads] beside a row arena, [arena_rows /
 * page_size, kv_heads, page_size] beside a page-tile arena). Queries stay
 * fp16. Other arguments as pda_rope_append. */
int pda_rope_append_q8(const void* q, void* q_out, const void* k, const void* v,
                       void* k_arena, void* v_arena, void* key_scales,
                       void* value_scales, const int32_t* positions,
                       const int32_t* rows, int32_t n, int32_t q_heads,
                       int32_t kv_heads, int32_t head_dim, int32_t page_size,
                       int64_t arena_rows, int32_t layout, int32_t rope_dims,
                       const float* inv_freq, void* stream);

/* Device-side packing of one decode step's page tables. Replaces the host
 * packing of DecodeBatch.__init__ (batches.py:148-179: tables [B, width] int32
 * with 0 padding, lengths = positions + 1, write rows table[pos / P] * P +
 * pos % P) for an engine that keeps every request's page list resident on the
 * device: seq_tables [num_slots, seq_stride] int32 holds request slot s's
 * physical pages in row s. For each sequence b of the step (request slot
 * slots[b], new token at positions[b]) it writes
 *   tables[b][j]  = seq_tables[slots[b]][j] for j <= positions[b] / page_size,
 *                   0 for the other j < width;
 *   lengths[b]    = positions[b] + 1;
 *   rows[b]       = tables[b][positions[b] / page_size] * page_size +
 *                   positions[b] % page_size, or -1 when that page index is
 *                   not below width and seq_stride.
 * A slot outside [0, num_slots) or a negative position gives a zero row,
 * length 0 and row -1. One launch on `stream`, no workspace; it can be
 * captured in a HIP graph with the decode calls that read its outputs. */
int pda_pack_decode_step(const int32_t* seq_tables, int32_t seq_stride,
                         int32_t num_slots, const int32_t* slots,
                         const int32_t* positions, int32_t batch, int32_t width,
                         int32_t page_size, int32_t* tables, int32_t* lengths,
                         int32_t* rows, void* stream);

/* Key ranges and workspace of a prefill call (pda_paged_prefill_attention
 * with the same start, count, q_heads, head_dim, window and splits).
 * `splits` 0 lets the library choose: 1 when the chunk's query tiles and
 * heads alone fill the GPU, else enough ranges to do so (a 512-token chunk
 * over a long prefix, the reference's default prefill chunk,
 * mlx_engine.py:74,430). `splits` > 0 forces that many (at most 64).
 * Writes the count used to *splits_used (may be NULL) and the bytes to
 * *bytes (0 for one range). No counterpart in the reference, whose prefill
 * attention is one MLX call per chunk. */
int pda_prefill_workspace_bytes(int32_t start, int32_t count, int32_t q_heads,
                                int32_t head_dim, int32_t window, int32_t splits,
                                int32_t* splits_used, size_t* bytes);

/* Paged prefill attention for a chunk of one sequence's prompt. Replaces
 * PrefillBatch.attend's attention (batches.py:84-132; CUDA analogue
 * cuda/kernels.cu:260-304) after the chunk's keys and values were written
 * (pda_rope_append with n = count):
 *   queries, out  [count, q_heads, head_dim] fp16, the chunk's tokens at
 *                 positions start .. start + count - 1 (queries rotated)
 *   keys, values  one layer's fp16 arena (layout as for the decode call)
 *   table         [table_len] int32, the sequence's physical pages
 *                 (table_len >= 1)
 * Query p attends keys [first(p), p]: first(p) = max(0, p - window + 1) with
 * a window, else 0; keys on a page id that is negative, not below
 * arena_rows / page_size or past table_len are masked (the reference raises
 * on released pages in range). The score is scale * q.k, softcapped when
 * softcap > 0. `images` (device int32 [num_images, 2], may be NULL when
 * num_images is 0) lists image-token spans [begin, end) of positions: a
 * query inside a span also sees every key of that span up to the chunk's
 * end, whatever the causal limit and the window (batches.py:107-118).
 * Any head_dim up to 512, as for the decode call: 64, 96, 128, 256 and 512
 * (the 512-wide heads of Gemma 4's global layers, docs/roadmap.md:36) run
 * kernels of their own, the others the next wider one with the dims past
 * head_dim zero (odd ones moving single elements); larger head dims return
 * PDA_ERR_HEAD_DIM.
 * With more than one key range
 * (see pda_prefill_workspace_bytes; results do not depend on `splits`
 * beyond fp32 rounding) the ranges' partials go to `workspace` (256-byte
 * aligned, at least the bytes that call reports) and a second launch merges
 * them; else one launch and no workspace. Both on `stream`. */
int pda_paged_prefill_attention(const void* queries, const void* keys,
                                const void* values, const int32_t* table,
                                int32_t table_len, int32_t start, int32_t count,
                                void* out, int32_t q_heads, int32_t kv_heads,
                                int32_t head_dim, int32_t page_size,
                                int64_t arena_rows, int32_t layout, float scale,
                                int32_t window, float softcap,
                                const int32_t* images, int32_t num_images,
                                int32_t splits, void* workspace,
                                size_t workspace_bytes, void* stream);

/* bf16 models: pda_paged_prefill_attention with queries, K/V arenas and
 * output in bf16 (KVCache(dtype=bfloat16), paged_kv.py:156-166). Scores and
 * the output accumulate in float32 on the bf16 matrix cores; the
 * probabilities that weight V are rounded to bf16 and the output to bf16 to
 * nearest even. Arguments and workspace as pda_paged_prefill_attention. */
int pda_paged_prefill_attention_bf16(const void* queries, const void* keys,
                                     const void* values, const int32_t* table,
                                     int32_t table_len, int32_t start, int32_t count,
                                     void* out, int32_t q_heads, int32_t kv_heads,
                                     int32_t head_dim, int32_t page_size,
                                     int64_t arena_rows, int32_t layout, float scale,
                                     int32_t window, float softcap,
                                     const int32_t* images, int32_t num_images,
                                     int32_t splits, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* Paged prefill attention over an 8-bit K/V cache. Replaces
 * PrefillBatch.attend's attention with KVCache(bits=8) (batches.py:84-132,
 * whose gather dequantizes, paged_kv.py:285-292): the arguments of
 * pda_paged_prefill_attention with int8 `keys`/`values` and their fp16 scale
 * arenas after `values` ([rows, kv_heads] beside the row arena,
 * [pages, kv_heads, page_size] beside page tiles, as for
 * pda_paged_decode_attention_q8). Each row is dequantized to
 * fp16(int8 x scale) as the reference's gather does, then attended as in
 * the fp16 call; the same workspace sizing (pda_prefill_workspace_bytes). */
int pda_paged_prefill_attention_q8(const void* queries, const void* keys,
                                   const void* values, const void* key_scales,
                                   const void* value_scales, const int32_t* table,
                                   int32_t table_len, int32_t start, int32_t count,
                                   void* out, int32_t q_heads, int32_t kv_heads,
                                   int32_t head_dim, int32_t page_size,
                                   int64_t arena_rows, int32_t layout, float scale,
                                   int32_t window, float softcap,
                                   const int32_t* images, int32_t num_images,
                                   int32_t splits, void* workspace,
                                   size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PDA_H */
