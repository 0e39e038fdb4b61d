// Sanitizer driver for the oracle's C++ restatement (oracle/cpu_attention.cpp,
// built with AddressSanitizer and UndefinedBehaviorSanitizer). It runs both
// decode restatements over small seeded batches that hold every edge the
// decode call defines: lengths of 0, negative lengths, lengths above
// table_stride x page_size (clamped), released (-1) and out-of-arena pages,
// windows wider and narrower than a sequence, softcap, one and four
// threads, and forced split counts above the number of keys. The float32
// split-K result must agree with the float64 one; the half conversions must
// round-trip every fp16 bit pattern.
//
// Exit status 0 when every check holds; sanitizer findings abort the run.

#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <random>
#include <vector>

extern "C" {
int oracle_version(void);
void oracle_half_to_float(const uint16_t* in, float* out, int64_t n);
void oracle_float_to_half(const float* in, uint16_t* out, int64_t n);
void oracle_decode_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const int32_t* tables, const int32_t* lengths, double* out, int B,
                       int HQ, int HKV, int D, int P, int stride, int64_t arena_rows,
                       double scale, int window, double softcap, int threads);
void oracle_decode_splitk(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                          const int32_t* tables, const int32_t* lengths, uint16_t* out, int B,
                          int HQ, int HKV, int D, int P, int stride, int64_t arena_rows,
                          float scale, int window, float softcap, int splits, int threads);
}

namespace {

int failures = 0;

void expect(bool ok, const char* what, int line) {
  if (!ok) {
    fprintf(stderr, "FAILED line %d: %s\n", line, what);
    ++failures;
  }
}
#define EXPECT(x) expect((x), #x, __LINE__)

void half_round_trip() {
  std::vector<uint16_t> bits(65536), back(65536);
  std::vector<float> f(65536);
  for (int i = 0; i < 65536; ++i) bits[i] = (uint16_t)i;
  oracle_half_to_float(bits.data(), f.data(), 65536);
  oracle_float_to_half(f.data(), back.data(), 65536);
  int bad = 0;
  for (int i = 0; i < 65536; ++i) {
    if (isnan(f[i]))
      bad += (back[i] & 0x7c00) != 0x7c00 || !(back[i] & 0x3ff);  // still a NaN
    else
      bad += back[i] != bits[i];
  }
  EXPECT(bad == 0);
}

struct Case {
  int B, HQ, HKV, D, P, stride, pages;
  int window;
  float softcap;
  std::vector<int32_t> lengths;
  std::vector<int> released;  // table entries set to -1 (b * stride + j)
  std::vector<int> outside;   // table entries set past the arena
};

void run(const Case& c, uint32_t seed) {
  std::mt19937 rng(seed);
  std::normal_distribution<float> normal(0.0f, 1.0f);
  const int64_t rows = (int64_t)c.pages * c.P;
  std::vector<float> qf((size_t)c.B * c.HQ * c.D), kf((size_t)rows * c.HKV * c.D),
      vf((size_t)rows * c.HKV * c.D);
  for (auto* x : {&qf, &kf, &vf})
    for (float& e : *x) e = normal(rng);
  std::vector<uint16_t> q(qf.size()), k(kf.size()), v(vf.size());
  oracle_float_to_half(qf.data(), q.data(), (int64_t)q.size());
  oracle_float_to_half(kf.data(), k.data(), (int64_t)k.size());
  oracle_float_to_half(vf.data(), v.data(), (int64_t)v.size());
  std::vector<int32_t> tables((size_t)c.B * c.stride);
  for (auto& t : tables) t = (int32_t)(rng() % c.pages);
  for (int i : c.released) tables[i] = -1;
  for (int i : c.outside) tables[i] = c.pages + 3;
  const double scale = 1.0 / sqrt((double)c.D);
  std::vector<double> ref((size_t)c.B * c.HQ * c.D, -1.0);
  for (int threads : {1, 4}) {
    oracle_decode_f64(q.data(), k.data(), v.data(), tables.data(), c.lengths.data(), ref.data(),
                      c.B, c.HQ, c.HKV, c.D, c.P, c.stride, rows, scale, c.window, c.softcap,
                      threads);
    for (int splits : {0, 1, 3, 97}) {
      std::vector<uint16_t> out(ref.size(), 0xffff);
      oracle_decode_splitk(q.data(), k.data(), v.data(), tables.data(), c.lengths.data(),
                           out.data(), c.B, c.HQ, c.HKV, c.D, c.P, c.stride, rows, (float)scale,
                           c.window, c.softcap, splits, threads);
      std::vector<float> got(out.size());
      oracle_half_to_float(out.data(), got.data(), (int64_t)out.size());
      double worst = 0.0;
      for (size_t i = 0; i < got.size(); ++i) {
        EXPECT(isfinite(got[i]) && isfinite(ref[i]));
        worst = fmax(worst, fabs(got[i] - ref[i]));
      }
      EXPECT(worst <= 2e-3);
    }
  }
  // A sequence with no visible key gives a zero row.
  for (int b = 0; b < c.B; ++b)
    if (c.lengths[b] <= 0)
      for (int i = 0; i < c.HQ * c.D; ++i) EXPECT(ref[(size_t)b * c.HQ * c.D + i] == 0.0);
}

}  // namespace

int main() {
  EXPECT(oracle_version() == 1);
  half_round_trip();
  // Lengths: empty, negative, one key, a page plus one, clamped to the
  // stride, and long; pages released before the window and off the arena.
  run({5, 8, 2, 64, 16, 8, 40, 0, 0.0f, {0, -3, 1, 17, 1000}, {}, {}}, 1);
  run({3, 6, 3, 36, 5, 30, 50, 20, 0.0f, {149, 21, 7}, {0, 1, 30, 31}, {}}, 2);
  run({4, 12, 4, 80, 16, 12, 60, 0, 30.0f, {190, 60, 5, 0}, {}, {3, 14, 37}}, 3);
  run({2, 2, 1, 4, 2, 2, 4, 0, 0.0f, {3, 4}, {}, {}}, 4);
  run({2, 16, 1, 512, 1, 40, 48, 7, 0.0f, {40, 9}, {0, 1}, {}}, 5);
  printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
