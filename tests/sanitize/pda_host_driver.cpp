// Host-side sanitizer driver for libpda's C-ABI (built with AddressSanitizer
// and UndefinedBehaviorSanitizer, device code not built). It runs the host
// code every call runs before its first HIP call: argument validation, the
// split planner, workspace layouts and the prefill range planner, over
// sweeps of shapes that include the extremes (lengths up to 2^31 - 1,
// batch 8184, every head dim up to 514, page sizes 1 .. 2^16) and every
// rejected argument. Calls with valid arguments reach HIP only when no GPU
// is visible (they then return PDA_ERR_HIP); with a GPU present the driver
// makes no such call, since its buffers are host memory.
//
// Exit status 0 when every call returned what the header documents;
// sanitizer findings abort the run (halt_on_error).

#include <hip/hip_runtime_api.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <thread>
#include <vector>

#include "pda.h"

namespace {

int failures = 0;

void expect(bool ok, const char* what, int line) {
  if (!ok) {
    fprintf(stderr, "FAILED line %d: %s (last error: %s)\n", line, what, pda_last_error());
    ++failures;
  }
}
#define EXPECT(x) expect((x), #x, __LINE__)

// Host buffers standing in for device pointers: 256-byte aligned, never
// dereferenced by the host code (the sanitizer would report it if they were).
alignas(256) char pool[1 << 16];
void* buf(int off = 0) { return pool + off; }
int32_t* ibuf(int off = 0) { return reinterpret_cast<int32_t*>(pool + off); }

bool no_gpu() {
  int n = 0;
  return hipGetDeviceCount(&n) != hipSuccess || n == 0;
}

void planner_sweep() {
  const int32_t batches[] = {1, 2, 7, 64, 1000, 8184, 8185, 0, -1};
  const int32_t heads[][2] = {{1, 1}, {8, 1}, {28, 4}, {64, 8}, {128, 1}, {40, 2}, {6, 4},
                              {0, 1}, {8, 0}};
  const int32_t dims[] = {2, 4, 64, 80, 96, 100, 128, 200, 256, 510, 512, 0, 7, 514, -2};
  const int32_t pages[] = {1, 3, 16, 128, 65536, 0};
  const int32_t lengths[] = {0, 1, 100, 32768, 1 << 20, 2147483647, -5};
  const int32_t windows[] = {0, 1, 4096, -1};
  const int32_t splits[] = {0, 1, 5, -1};
  int calls = 0, planned = 0;
  for (int32_t b : batches)
    for (auto& h : heads)
      for (int32_t d : dims)
        for (int32_t p : pages)
          for (int32_t n : lengths)
            for (int32_t w : windows)
              for (int32_t sp : splits) {
                const int32_t stride = p > 0 && n > 0 ? (int32_t)((int64_t)n / p + 1) : 4;
                size_t bytes = 1;
                const int rc = pda_workspace_bytes(b, h[0], h[1], d, p, stride, n, w, sp, &bytes);
                int32_t waves = -1, per = -1;
                const int rc2 = pda_plan(b, h[0], h[1], d, p, stride, n, w, sp, &waves, &per);
                ++calls;
                EXPECT(rc == rc2);
                EXPECT(rc == PDA_OK || rc == PDA_ERR_INVALID_ARGUMENT ||
                       rc == PDA_ERR_HEAD_RATIO || rc == PDA_ERR_HEAD_DIM ||
                       rc == PDA_ERR_TOO_LONG);
                if (rc == PDA_OK) {
                  ++planned;
                  EXPECT(bytes > 0 && bytes % 256 == 0);
                  EXPECT(waves >= 1 && per >= 0);  // 0 pages: nothing visible
                }
              }
  EXPECT(planned > 0);
  printf("planner: %d shapes, %d planned\n", calls, planned);
  // Null outputs are rejected.
  EXPECT(pda_workspace_bytes(1, 8, 1, 128, 16, 4, 10, 0, 0, nullptr) ==
         PDA_ERR_INVALID_ARGUMENT);
}

void prefill_planner_sweep() {
  const int32_t starts[] = {0, 1, 500, 4096, 1 << 20, 2147483647 - 600, -1};
  const int32_t counts[] = {0, 1, 100, 512, 4096, 1 << 16, -1};
  const int32_t heads[] = {1, 8, 28, 128, 0};
  const int32_t dims[] = {2, 4, 64, 80, 96, 128, 130, 256, 510, 512, 0, 1, 514};
  const int32_t windows[] = {0, 1, 256, -1};
  const int32_t splits[] = {0, 1, 3, 64, 500, -1};
  int calls = 0;
  for (int32_t s : starts)
    for (int32_t c : counts)
      for (int32_t h : heads)
        for (int32_t d : dims)
          for (int32_t w : windows)
            for (int32_t sp : splits) {
              int32_t used = -1;
              size_t bytes = 1;
              const int rc = pda_prefill_workspace_bytes(s, c, h, d, w, sp, &used, &bytes);
              ++calls;
              EXPECT(rc == PDA_OK || rc == PDA_ERR_INVALID_ARGUMENT || rc == PDA_ERR_HEAD_DIM);
              if (rc == PDA_OK) {
                EXPECT(used >= 1 && used <= 64);
                EXPECT(bytes % 256 == 0 && (used > 1) == (bytes > 0));
              }
            }
  EXPECT(pda_prefill_workspace_bytes(0, 10, 8, 64, 0, 0, nullptr, nullptr) ==
         PDA_ERR_INVALID_ARGUMENT);
  printf("prefill planner: %d shapes\n", calls);
}

// The decode entry points with one bad argument each: every one is rejected
// on the host.
typedef int (*DecodeFn)(const void*, const void*, const void*, const int32_t*, const int32_t*,
                        void*, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int64_t,
                        int32_t, int32_t, float, int32_t, float, int32_t, int32_t, void*, size_t,
                        void*);

struct DecodeArgs {
  const void* q = buf(0);
  const void* k = buf(4096);
  const void* v = buf(8192);
  const int32_t* tables = ibuf(12288);
  const int32_t* lengths = ibuf(16384);
  void* out = buf(20480);
  int32_t batch = 4, hq = 28, hkv = 4, d = 128, page = 16, stride = 64;
  int64_t rows = 4096;
  int32_t layout = PDA_LAYOUT_PAGES, longest = 1000;
  float scale = 0.088f;
  int32_t window = 0;
  float softcap = 0.0f;
  int32_t split_pages = 0, flags = 0;
  void* ws = buf(32768);
  size_t ws_bytes = 1 << 30;
  int call(DecodeFn f) const {
    return f(q, k, v, tables, lengths, out, batch, hq, hkv, d, page, stride, rows, layout,
             longest, scale, window, softcap, split_pages, flags, ws, ws_bytes, nullptr);
  }
};

void decode_validation(bool may_reach_hip) {
  const DecodeFn fns[] = {pda_paged_decode_attention, pda_decode_split, pda_decode_merge,
                          pda_paged_decode_attention_bf16, pda_decode_split_bf16,
                          pda_decode_merge_bf16};
  for (DecodeFn f : fns) {
    struct Bad {
      void (*set)(DecodeArgs&);
      int code;
    };
    const Bad bad[] = {
        {[](DecodeArgs& a) { a.q = nullptr; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.out = nullptr; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.batch = -1; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.batch = 9000; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.hq = 30; }, PDA_ERR_HEAD_RATIO},
        {[](DecodeArgs& a) { a.d = 513; }, PDA_ERR_HEAD_DIM},
        {[](DecodeArgs& a) { a.d = 514; }, PDA_ERR_HEAD_DIM},
        {[](DecodeArgs& a) { a.page = 0; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.layout = 2; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.rows = 8; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.q = buf(8); }, PDA_ERR_ALIGNMENT},
        {[](DecodeArgs& a) { a.tables = ibuf(2); }, PDA_ERR_ALIGNMENT},
        {[](DecodeArgs& a) { a.ws = nullptr; }, PDA_ERR_WORKSPACE},
        {[](DecodeArgs& a) { a.ws_bytes = 1024; }, PDA_ERR_WORKSPACE},
        {[](DecodeArgs& a) { a.ws = buf(32768 + 16); }, PDA_ERR_ALIGNMENT},
        {[](DecodeArgs& a) { a.scale = 0.0f / 0.0f; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.softcap = -1.0f; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.flags = 4; }, PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.flags = PDA_DECODE_FIXED_SPLIT | PDA_DECODE_RACING; },
         PDA_ERR_INVALID_ARGUMENT},
        {[](DecodeArgs& a) { a.window = -1; }, PDA_ERR_INVALID_ARGUMENT},
    };
    for (const Bad& b : bad) {
      DecodeArgs a;
      b.set(a);
      const int rc = a.call(f);
      EXPECT(rc == b.code);
      EXPECT(strlen(pda_last_error()) > 0);
    }
    if (may_reach_hip) {
      DecodeArgs a;
      EXPECT(a.call(f) == PDA_ERR_HIP);
      a.d = 80;
      a.flags = PDA_DECODE_FIXED_SPLIT;
      EXPECT(a.call(f) == PDA_ERR_HIP);
      a.flags = PDA_DECODE_RACING;
      EXPECT(a.call(f) == PDA_ERR_HIP);
    }
  }
  // 8-bit: its scale arenas.
  for (int which = 0; which < 3; ++which) {
    DecodeArgs a;
    const void* ks = buf(40960);
    const void* vs = which == 1 ? nullptr : buf(which == 2 ? 40961 : 45056);
    int (*f)(const void*, const void*, const void*, const void*, const void*, const int32_t*,
             const int32_t*, void*, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t,
             int64_t, int32_t, int32_t, float, int32_t, float, int32_t, int32_t, void*, size_t,
             void*) = pda_paged_decode_attention_q8;
    const int rc = f(a.q, a.k, a.v, ks, vs, a.tables, a.lengths, a.out, a.batch, a.hq, a.hkv,
                     a.d, a.page, a.stride, a.rows, a.layout, a.longest, a.scale, a.window,
                     a.softcap, a.split_pages, a.flags, a.ws, a.ws_bytes, nullptr);
    if (which == 1) EXPECT(rc == PDA_ERR_INVALID_ARGUMENT);
    if (which == 2) EXPECT(rc == PDA_ERR_ALIGNMENT);
    if (which == 0 && may_reach_hip) EXPECT(rc == PDA_ERR_HIP);
  }
  // The call without a workspace: valid shapes reach HIP (the static
  // scratch's address), bad ones do not.
  {
    DecodeArgs a;
    const int rc = pda_paged_decode_attention_noalloc(
        a.q, a.k, a.v, a.tables, a.lengths, a.out, a.batch, a.hq, 1, a.d, a.page, a.stride,
        a.rows, a.layout, a.longest, a.scale, a.window, a.softcap, 0, 0, nullptr);
    EXPECT(rc == PDA_ERR_HEAD_RATIO || rc == PDA_OK || rc == PDA_ERR_HIP);
    EXPECT(pda_paged_decode_attention_noalloc(a.q, a.k, a.v, a.tables, a.lengths, a.out, -1,
                                              a.hq, a.hkv, a.d, a.page, a.stride, a.rows,
                                              a.layout, a.longest, a.scale, a.window,
                                              a.softcap, 0, 0, nullptr) ==
           PDA_ERR_INVALID_ARGUMENT);
    // An empty batch is a no-op on every decode entry point.
    a.batch = 0;
    EXPECT(a.call(pda_paged_decode_attention) == PDA_OK);
  }
}

void prefill_validation(bool may_reach_hip) {
  typedef int (*PrefillFn)(const void*, const void*, const void*, const int32_t*, int32_t,
                           int32_t, int32_t, void*, int32_t, int32_t, int32_t, int32_t,
                           int64_t, int32_t, float, int32_t, float, const int32_t*, int32_t,
                           int32_t, void*, size_t, void*);
  const PrefillFn fns[] = {pda_paged_prefill_attention, pda_paged_prefill_attention_bf16};
  for (PrefillFn f : fns) {
    auto call = [&](int32_t count, int32_t hq, int32_t hd, int32_t page, int32_t splits,
                    void* ws, size_t ws_bytes, const void* q, int32_t num_images,
                    const int32_t* images, int32_t start = 300, int32_t table_len = 64) {
      return f(q, buf(4096), buf(8192), ibuf(12288), table_len, start, count, buf(20480), hq,
               4, hd, page, 4096, PDA_LAYOUT_ROWS, 0.1f, 0, 0.0f, images, num_images, splits,
               ws, ws_bytes, nullptr);
    };
    EXPECT(call(0, 28, 128, 16, 0, nullptr, 0, nullptr, 0, nullptr) == PDA_OK);
    EXPECT(call(-1, 28, 128, 16, 0, nullptr, 0, buf(), 0, nullptr) == PDA_ERR_INVALID_ARGUMENT);
    EXPECT(call(10, 30, 128, 16, 0, nullptr, 0, buf(), 0, nullptr) == PDA_ERR_HEAD_RATIO);
    EXPECT(call(10, 28, 513, 16, 0, nullptr, 0, buf(), 0, nullptr) == PDA_ERR_HEAD_DIM);
    EXPECT(call(10, 28, 0, 16, 0, nullptr, 0, buf(), 0, nullptr) == PDA_ERR_HEAD_DIM);
    EXPECT(call(10, 28, 128, 0, 0, nullptr, 0, buf(), 0, nullptr) == PDA_ERR_INVALID_ARGUMENT);
    EXPECT(call(10, 28, 128, 16, 4, nullptr, 0, buf(), 0, nullptr) == PDA_ERR_WORKSPACE);
    EXPECT(call(10, 28, 128, 16, 0, nullptr, 0, buf(8), 0, nullptr) == PDA_ERR_ALIGNMENT);
    EXPECT(call(10, 28, 128, 16, 0, nullptr, 0, buf(), 2, nullptr) == PDA_ERR_INVALID_ARGUMENT);
    EXPECT(call(10, 28, 128, 16, 0, nullptr, 0, buf(), 1, ibuf(2)) == PDA_ERR_ALIGNMENT);
    EXPECT(call(10, 28, 128, 16, 0, nullptr, 0, buf(), 0, nullptr, 2147483647 - 5) ==
           PDA_ERR_TOO_LONG);
    EXPECT(call(10, 28, 128, 16, 0, nullptr, 0, buf(), 0, nullptr, 300, 0) ==
           PDA_ERR_INVALID_ARGUMENT);
    if (may_reach_hip) {
      for (int32_t hd : {4, 80, 128, 200, 512})
        for (int32_t splits : {1, 3})
          EXPECT(call(100, 28, hd, 16, splits, buf(32768), (size_t)1 << 30, buf(), 0,
                      nullptr) == PDA_ERR_HIP);
    }
  }
}

void append_and_pack_validation(bool may_reach_hip) {
  const float* inv = reinterpret_cast<const float*>(buf(24576));
  EXPECT(pda_rope_append(buf(), buf(256), buf(512), buf(768), buf(4096), buf(8192), ibuf(12288),
                         ibuf(12544), 4, 28, 4, 128, 16, 4096, PDA_LAYOUT_ROWS, 130, inv,
                         nullptr) == PDA_ERR_INVALID_ARGUMENT);  // rope_dims > head_dim
  EXPECT(pda_rope_append(buf(), buf(256), buf(512), buf(768), buf(4096), buf(8192), ibuf(12288),
                         ibuf(12544), 4, 28, 4, 600, 16, 4096, PDA_LAYOUT_ROWS, 0, inv,
                         nullptr) != PDA_OK);  // head_dim above 512
  EXPECT(pda_rope_append(nullptr, buf(256), buf(512), buf(768), buf(4096), buf(8192),
                         ibuf(12288), ibuf(12544), 4, 28, 4, 128, 16, 4096, PDA_LAYOUT_ROWS,
                         128, inv, nullptr) == PDA_ERR_INVALID_ARGUMENT);
  EXPECT(pda_pack_decode_step(ibuf(0), 64, 8, ibuf(4096), ibuf(8192), 4, 0, 16, ibuf(12288),
                              ibuf(16384), ibuf(20480), nullptr) == PDA_ERR_INVALID_ARGUMENT);
  EXPECT(pda_pack_decode_step(ibuf(0), 64, 8, nullptr, ibuf(8192), 4, 32, 16, ibuf(12288),
                              ibuf(16384), ibuf(20480), nullptr) == PDA_ERR_INVALID_ARGUMENT);
  if (may_reach_hip) {
    EXPECT(pda_rope_append(buf(), buf(256), buf(512), buf(768), buf(4096), buf(8192),
                           ibuf(12288), ibuf(12544), 4, 28, 4, 80, 16, 4096, PDA_LAYOUT_PAGES,
                           80, inv, nullptr) == PDA_ERR_HIP);
    EXPECT(pda_pack_decode_step(ibuf(0), 64, 8, ibuf(4096), ibuf(8192), 4, 32, 16, ibuf(12288),
                                ibuf(16384), ibuf(20480), nullptr) == PDA_ERR_HIP);
  }
}

void last_error_is_per_thread() {
  DecodeArgs a;
  a.d = 513;
  EXPECT(a.call(pda_paged_decode_attention) == PDA_ERR_HEAD_DIM);
  const std::string mine = pda_last_error();
  std::string theirs = "unset";
  std::thread t([&] {
    DecodeArgs b;
    b.hq = 30;
    b.call(pda_paged_decode_attention);
    theirs = pda_last_error();
  });
  t.join();
  EXPECT(mine == pda_last_error());
  EXPECT(theirs != mine && !theirs.empty());
  size_t bytes = 0;
  EXPECT(pda_workspace_bytes(1, 8, 1, 128, 16, 4, 10, 0, 0, &bytes) == PDA_OK);
  EXPECT(strlen(pda_last_error()) == 0);
}

}  // namespace

int main() {
  const bool cpu_only = no_gpu();
  printf("libpda %d.%d, %s\n", pda_version() >> 16, pda_version() & 0xffff,
         cpu_only ? "no GPU: valid calls reach HIP" : "GPU present: validation only");
  planner_sweep();
  prefill_planner_sweep();
  decode_validation(cpu_only);
  prefill_validation(cpu_only);
  append_and_pack_validation(cpu_only);
  last_error_is_per_thread();
  printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
