// CPU restatement of the reference's paged decode attention — TEST
// INFRASTRUCTURE ONLY (the checker and the timed CPU baseline). Only tests/,
// __graft_entry__.smoke() and bench.py's CPU-baseline leg load it.
//
// Three entry points, each threaded over (sequence, kv head[, split]) with
// std::thread on the cores they are given:
//
//  oracle_decode_f64    The portable ("MLX CPU") decode path: gather the
//                       visible rows through the page table, mask released
//                       pages, dense softmax(q.K^T * scale) @ V with every
//                       product and sum in float64.
//                       python/instinct/backends/portable.py:155-205 and
//                       python/instinct/batches.py:183-189,228-246.
//  oracle_decode_f32    The same portable path in float32, as the reference
//                       computes it (_attention_plain: float32 scores,
//                       softmax and product, fp16 output): the timed CPU
//                       baseline.
//  oracle_decode_splitk The Metal kernel's split-K algorithm in float32:
//                       per (sequence, kv head, split) the per-key online
//                       softmax update, unnormalised partials, then the
//                       log-sum-exp merge; fp16 output.
//                       python/instinct/backends/metal_kernels.py:18-124,
//                       split rule :126-127,193-194.
//
// Layouts follow pda.h: q [B,HQ,D] fp16, keys/values [rows,HKV,D] fp16,
// tables [B,stride] int32, lengths [B] int32. fp16 values travel as uint16
// bit patterns.

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const uint32_t exp = (h >> 10) & 0x1F;
  const uint32_t man = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: renormalise
      int e = -1;
      uint32_t m = man;
      do {
        ++e;
        m <<= 1;
      } while ((m & 0x400) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3FF) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Round-to-nearest-even float -> fp16 bits.
uint16_t float_to_half(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  const uint32_t absx = x & 0x7FFFFFFFu;
  if (absx >= 0x7F800000u)  // inf or nan
    return sign | 0x7C00 | (absx > 0x7F800000u ? 0x200 : 0);
  if (absx >= 0x477FF000u) return sign | 0x7C00;  // rounds to inf
  if (absx < 0x38800000u) {                       // subnormal or zero
    if (absx < 0x33000000u) return sign;  // below 2^-25: rounds to zero
    const uint32_t e = absx >> 23;
    const uint32_t m = (absx & 0x7FFFFF) | 0x800000;  // value = m * 2^(e-150)
    // In units of the fp16 subnormal step 2^-24 the value is m >> (126 - e).
    const int s = 126 - (int)e;  // 14..24
    uint32_t r = m >> s;
    const uint32_t rem = m & ((1u << s) - 1);
    const uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (r & 1))) ++r;
    return sign | (uint16_t)r;
  }
  uint32_t r = ((absx >> 13) - ((127 - 15) << 10));
  const uint32_t rem = absx & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) ++r;
  return sign | (uint16_t)r;
}

struct Table16 {
  float v[65536];
  Table16() {
    for (uint32_t i = 0; i < 65536; ++i) v[i] = half_to_float((uint16_t)i);
  }
};
const Table16& tab() {
  static Table16 t;
  return t;
}

struct Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* tables;
  const int32_t* lengths;
  int B, HQ, HKV, D, P, stride;
  int64_t arena_rows;
  double scale;
  int window;
  double softcap;
};

// Visible positions [first, len) and their arena rows (-1 = masked).
void visible_rows(const Args& a, int b, int& first, int& len, std::vector<int64_t>& rows) {
  len = std::min<int64_t>(std::max(a.lengths[b], 0), (int64_t)a.stride * a.P);
  first = a.window > 0 ? std::max(0, len - a.window) : 0;
  rows.resize(std::max(0, len - first));
  const int64_t pages = a.arena_rows / a.P;
  for (int t = first; t < len; ++t) {
    const int32_t page = a.tables[(int64_t)b * a.stride + t / a.P];
    rows[t - first] = (page >= 0 && page < pages) ? (int64_t)page * a.P + t % a.P : -1;
  }
}

template <class F>
void parallel_for(int64_t n, int threads, F fn) {
  threads = std::max(1, threads);
  std::atomic<int64_t> next(0);
  auto worker = [&]() {
    for (int64_t i; (i = next.fetch_add(1)) < n;) fn(i);
  };
  std::vector<std::thread> pool;
  for (int t = 1; t < threads; ++t) pool.emplace_back(worker);
  worker();
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

int oracle_version(void) { return 1; }

void oracle_half_to_float(const uint16_t* in, float* out, int64_t n) {
  const float* t = tab().v;
  for (int64_t i = 0; i < n; ++i) out[i] = t[in[i]];
}

void oracle_float_to_half(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = float_to_half(in[i]);
}

// Float64 dense oracle: out [B, HQ, D] float64.
void oracle_decode_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const int32_t* tables, const int32_t* lengths, double* out,
                       int B, int HQ, int HKV, int D, int P, int stride,
                       int64_t arena_rows, double scale, int window, double softcap,
                       int threads) {
  const Args a{q, k, v, tables, lengths, B, HQ, HKV, D, P, stride, arena_rows, scale, window, softcap};
  const int G = HQ / HKV;
  const float* t16 = tab().v;
  parallel_for((int64_t)B * HKV, threads, [&](int64_t item) {
    const int b = (int)(item / HKV), kvh = (int)(item % HKV);
    int first, len;
    std::vector<int64_t> rows;
    visible_rows(a, b, first, len, rows);
    const int n = (int)rows.size();
    std::vector<double> qd((size_t)G * D), s((size_t)G * n), acc((size_t)G * D, 0.0);
    for (int g = 0; g < G; ++g)
      for (int d = 0; d < D; ++d)
        qd[(size_t)g * D + d] = t16[q[((int64_t)b * HQ + kvh * G + g) * D + d]];
    std::vector<double> kr(D);
    for (int i = 0; i < n; ++i) {
      if (rows[i] < 0) {
        for (int g = 0; g < G; ++g) s[(size_t)g * n + i] = -INFINITY;
        continue;
      }
      const uint16_t* kp = k + (rows[i] * HKV + kvh) * D;
      for (int d = 0; d < D; ++d) kr[d] = t16[kp[d]];
      for (int g = 0; g < G; ++g) {
        double dot = 0.0;
        for (int d = 0; d < D; ++d) dot += qd[(size_t)g * D + d] * scale * kr[d];
        if (softcap > 0.0) dot = std::tanh(dot / softcap) * softcap;
        s[(size_t)g * n + i] = dot;
      }
    }
    std::vector<double> top(G, -INFINITY), sum(G, 0.0);
    for (int g = 0; g < G; ++g)
      for (int i = 0; i < n; ++i) top[g] = std::max(top[g], s[(size_t)g * n + i]);
    std::vector<double> vr(D);
    for (int i = 0; i < n; ++i) {
      if (rows[i] < 0) continue;
      const uint16_t* vp = v + (rows[i] * HKV + kvh) * D;
      for (int d = 0; d < D; ++d) vr[d] = t16[vp[d]];
      for (int g = 0; g < G; ++g) {
        const double p = std::exp(s[(size_t)g * n + i] - top[g]);
        sum[g] += p;
        for (int d = 0; d < D; ++d) acc[(size_t)g * D + d] += p * vr[d];
      }
    }
    for (int g = 0; g < G; ++g)
      for (int d = 0; d < D; ++d)
        out[((int64_t)b * HQ + kvh * G + g) * D + d] =
            sum[g] > 0.0 ? acc[(size_t)g * D + d] / sum[g] : 0.0;
  });
}

// Float32 portable path (the "MLX CPU" decode the reference's engine runs
// without Metal kernels): gather the visible rows, then
// _attention_plain (portable.py:173-188) in float32: scores = (q * scale) .
// K^T, softcap, masked (released pages, portable.py:202-204), softmax
// (max, exp, sum, divide), probabilities @ V, cast to fp16. out [B, HQ, D]
// fp16 bits.
void oracle_decode_f32(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const int32_t* tables, const int32_t* lengths, uint16_t* out,
                       int B, int HQ, int HKV, int D, int P, int stride,
                       int64_t arena_rows, float scale, int window, float softcap,
                       int threads) {
  const Args a{q, k, v, tables, lengths, B, HQ, HKV, D, P, stride, arena_rows, scale, window, softcap};
  const int G = HQ / HKV;
  const float* t16 = tab().v;
  parallel_for((int64_t)B * HKV, threads, [&](int64_t item) {
    const int b = (int)(item / HKV), kvh = (int)(item % HKV);
    int first, len;
    std::vector<int64_t> rows;
    visible_rows(a, b, first, len, rows);
    const int n = (int)rows.size();
    // The gather: the visible K and V rows of this kv head, in float32.
    std::vector<float> kg((size_t)n * D), vg((size_t)n * D);
    for (int i = 0; i < n; ++i) {
      const int64_t r = rows[i] < 0 ? 0 : rows[i];
      const uint16_t* kp = k + (r * HKV + kvh) * D;
      const uint16_t* vp = v + (r * HKV + kvh) * D;
      for (int d = 0; d < D; ++d) kg[(size_t)i * D + d] = t16[kp[d]];
      for (int d = 0; d < D; ++d) vg[(size_t)i * D + d] = t16[vp[d]];
    }
    std::vector<float> qs(D), s(n), acc(D);
    for (int g = 0; g < G; ++g) {
      const int64_t h = (int64_t)b * HQ + kvh * G + g;
      for (int d = 0; d < D; ++d) qs[d] = t16[q[h * D + d]] * scale;
      float top = -INFINITY;
      for (int i = 0; i < n; ++i) {
        float dot = 0.0f;
        const float* kr = &kg[(size_t)i * D];
        for (int d = 0; d < D; ++d) dot += qs[d] * kr[d];
        if (softcap > 0.0f) dot = std::tanh(dot / softcap) * softcap;
        s[i] = rows[i] < 0 ? -INFINITY : dot;
        top = std::max(top, s[i]);
      }
      float sum = 0.0f;
      for (int i = 0; i < n; ++i) {
        s[i] = top == -INFINITY ? 0.0f : std::exp(s[i] - top);
        sum += s[i];
      }
      std::fill(acc.begin(), acc.end(), 0.0f);
      for (int i = 0; i < n; ++i) {
        const float p = sum > 0.0f ? s[i] / sum : 0.0f;
        const float* vr = &vg[(size_t)i * D];
        for (int d = 0; d < D; ++d) acc[d] += p * vr[d];
      }
      for (int d = 0; d < D; ++d) out[h * D + d] = float_to_half(acc[d]);
    }
  });
}

// Float32 split-K restatement of the Metal kernel; out [B, HQ, D] fp16 bits.
// splits <= 0 selects the reference rule clamp(ceil(span/512), 1, 128) from
// the longest visible span.
void oracle_decode_splitk(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          const int32_t* tables, const int32_t* lengths, uint16_t* out,
                          int B, int HQ, int HKV, int D, int P, int stride,
                          int64_t arena_rows, float scale, int window, float softcap,
                          int splits, int threads) {
  const int G = HQ / HKV;
  if (splits <= 0) {
    int longest = 0;
    for (int b = 0; b < B; ++b) longest = std::max(longest, lengths[b]);
    const int span = window > 0 ? std::min(longest, window) : longest;
    splits = std::max(1, std::min(128, (span + 511) / 512));
  }
  const int S = splits;
  const float* t16 = tab().v;
  std::vector<float> po((size_t)B * HQ * S * D), pm((size_t)B * HQ * S), pl((size_t)B * HQ * S);
  parallel_for((int64_t)B * HKV * S, threads, [&](int64_t item) {
    const int split = (int)(item % S);
    const int kvh = (int)((item / S) % HKV);
    const int b = (int)(item / ((int64_t)S * HKV));
    int len = std::min<int64_t>(std::max(lengths[b], 0), (int64_t)stride * P);
    const int first = window > 0 ? std::max(0, len - window) : 0;
    const int per = (len - first + S - 1) / S;
    const int begin = first + split * per;
    const int end = std::min(len, begin + per);
    const int64_t pages = arena_rows / P;
    std::vector<float> qf((size_t)G * D), o((size_t)G * D, 0.0f), kr(D), vr(D);
    std::vector<float> m(G, -INFINITY), l(G, 0.0f);
    for (int g = 0; g < G; ++g)
      for (int d = 0; d < D; ++d)
        qf[(size_t)g * D + d] = t16[q[((int64_t)b * HQ + kvh * G + g) * D + d]] * scale;
    for (int t = begin; t < end; ++t) {
      const int32_t page = tables[(int64_t)b * stride + t / P];
      if (page < 0 || page >= pages) continue;
      const int64_t row = (int64_t)page * P + t % P;
      const uint16_t* kp = k + (row * HKV + kvh) * D;
      const uint16_t* vp = v + (row * HKV + kvh) * D;
      for (int d = 0; d < D; ++d) kr[d] = t16[kp[d]];
      for (int d = 0; d < D; ++d) vr[d] = t16[vp[d]];
      for (int g = 0; g < G; ++g) {
        const float* qg = &qf[(size_t)g * D];
        float sc = 0.0f;
        for (int d = 0; d < D; ++d) sc += qg[d] * kr[d];
        if (softcap > 0.0f) sc = std::tanh(sc / softcap) * softcap;
        const float next = std::max(m[g], sc);
        const float factor = std::exp(m[g] - next);
        const float p = std::exp(sc - next);
        l[g] = l[g] * factor + p;
        float* og = &o[(size_t)g * D];
        for (int d = 0; d < D; ++d) og[d] = og[d] * factor + p * vr[d];
        m[g] = next;
      }
    }
    for (int g = 0; g < G; ++g) {
      const size_t slot = ((size_t)b * HQ + kvh * G + g) * S + split;
      std::memcpy(&po[slot * D], &o[(size_t)g * D], sizeof(float) * D);
      pm[slot] = m[g];
      pl[slot] = l[g];
    }
  });
  parallel_for((int64_t)B * HQ, threads, [&](int64_t bh) {
    float top = -INFINITY;
    for (int s = 0; s < S; ++s) top = std::max(top, pm[bh * S + s]);
    std::vector<float> acc(D, 0.0f);
    float total = 0.0f;
    for (int s = 0; s < S; ++s) {
      const float mm = pm[bh * S + s];
      if (mm == -INFINITY) continue;
      const float w = std::exp(mm - top);
      total += pl[bh * S + s] * w;
      const float* src = &po[((size_t)bh * S + s) * D];
      for (int d = 0; d < D; ++d) acc[d] += src[d] * w;
    }
    const float inv = total > 0.0f ? 1.0f / total : 0.0f;
    for (int d = 0; d < D; ++d) out[bh * D + d] = float_to_half(acc[d] * inv);
  });
}

}  // extern "C"
