// Device-side packing of a decode step's page tables, C-ABI in pda.h
// (pda_pack_decode_step).
//
// Reference step replaced: DecodeBatch.__init__ (python/instinct/
// batches.py:148-179) packs each request's page list into a [B, width] int32
// table with 0 padding in a Python loop, sets lengths = positions + 1 and the
// write rows table[pos // P] * P + pos % P, and uploads the three arrays every
// step (the host work docs/roadmap.md flags). Here the requests' page tables
// stay resident in device memory, one row per request slot, and one launch
// gathers the step's rows: nothing crosses PCIe and the launch can sit in a
// captured HIP graph with the attention launches of every layer.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "pda.h"
#include "pda_internal.h"

namespace {

constexpr int kPackThreads = 256;

struct PackParams {
  const int32_t* seq_tables;  // [num_slots, seq_stride] pages of each request slot
  const int32_t* slots;       // [batch] request slot of each sequence
  const int32_t* positions;   // [batch] position of the new token
  int32_t* tables;            // [batch, width] out
  int32_t* lengths;           // [batch] out
  int32_t* rows;              // [batch] out
  int32_t seq_stride;
  int32_t num_slots;
  int32_t width;
  int32_t page_size;
};

// Workgroup b packs sequence b: entries below the pages its length touches
// are copied, the rest are 0 (batches.py:171-174). A slot outside the table
// array or a negative position gives a zero row, length 0 and no write row.
__global__ __launch_bounds__(kPackThreads) void pack_decode_step_kernel(const PackParams p) {
  const int b = blockIdx.x;
  const int slot = p.slots[b];
  const int pos = p.positions[b];
  const bool ok = slot >= 0 && slot < p.num_slots && pos >= 0;
  const int used = ok ? min(pos / p.page_size + 1, p.seq_stride) : 0;
  const int32_t* src = p.seq_tables + (int64_t)(ok ? slot : 0) * p.seq_stride;
  int32_t* dst = p.tables + (int64_t)b * p.width;
  for (int j = threadIdx.x; j < p.width; j += kPackThreads) dst[j] = j < used ? src[j] : 0;
  if (threadIdx.x == 0) {
    const int page_index = ok ? pos / p.page_size : 0;
    const bool in_table = ok && page_index < p.seq_stride && page_index < p.width;
    p.lengths[b] = ok ? pos + 1 : 0;
    p.rows[b] = in_table ? src[page_index] * p.page_size + pos % p.page_size : -1;
  }
}

using pda_internal::fail;
using pda_internal::ok;

}  // namespace

extern "C" {

int pda_pack_decode_step(const int32_t* seq_tables, int32_t seq_stride, int32_t num_slots,
                         const int32_t* slots, const int32_t* positions, int32_t batch,
                         int32_t width, int32_t page_size, int32_t* tables,
                         int32_t* lengths, int32_t* rows, void* stream) {
  if (batch < 0 || seq_stride <= 0 || num_slots <= 0 || width <= 0 || page_size <= 0)
    return fail(PDA_ERR_INVALID_ARGUMENT,
                "batch=%d seq_stride=%d num_slots=%d width=%d page_size=%d", batch,
                seq_stride, num_slots, width, page_size);
  if (batch == 0) return ok();
  if (!seq_tables || !slots || !positions || !tables || !lengths || !rows)
    return fail(PDA_ERR_INVALID_ARGUMENT, "null buffer pointer");
  const uintptr_t mis = (uintptr_t)seq_tables | (uintptr_t)slots | (uintptr_t)positions |
                        (uintptr_t)tables | (uintptr_t)lengths | (uintptr_t)rows;
  if (mis & 3) return fail(PDA_ERR_ALIGNMENT, "int32 buffers must be 4-byte aligned");
  PackParams prm{seq_tables, slots,      positions, tables,     lengths,
                 rows,       seq_stride, num_slots, width,      page_size};
  void* args[] = {&prm};
  const hipError_t err =
      hipLaunchKernel(reinterpret_cast<const void*>(pack_decode_step_kernel), dim3(batch),
                      dim3(kPackThreads), args, 0, static_cast<hipStream_t>(stream));
  if (err != hipSuccess)
    return fail(PDA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

}  // extern "C"
