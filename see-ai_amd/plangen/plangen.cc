// plangen.cc -- bulk generation for the plan writer (see-ai_amd/planwriter.py):
// the deterministic N(0, std^2) weights and the per-column int8 packing of a
// frozen base, threaded.  Each function restates, element for element, the
// numpy definition in planwriter.py (normal(), quantize_cols()); the plan
// writer's tests hold the two to the same bytes.  Host code only, no GPU.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

namespace {

// SplitMix64 output `index` (1-based) from `seed`.
inline uint64_t SplitMix(uint64_t seed, uint64_t index) {
  uint64_t z = seed + index * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename F>
void Parallel(uint64_t n, uint64_t grain, F&& body) {
  const uint64_t chunks = (n + grain - 1) / grain;
  unsigned hw = std::thread::hardware_concurrency();
  const uint64_t workers = std::min<uint64_t>(chunks, std::clamp(hw, 1u, 16u));
  if (workers <= 1) {
    for (uint64_t c = 0; c < chunks; ++c) body(c * grain, std::min(n, (c + 1) * grain));
    return;
  }
  std::vector<std::thread> pool;
  for (uint64_t w = 0; w < workers; ++w)
    pool.emplace_back([&, w] {
      for (uint64_t c = w; c < chunks; c += workers) body(c * grain, std::min(n, (c + 1) * grain));
    });
  for (auto& t : pool) t.join();
}

}  // namespace

extern "C" {

// Pair p takes SplitMix outputs 2p+1 and 2p+2: u1 = ((x1 >> 11) + 1) 2^-53,
// u2 = (x2 >> 11) 2^-53, r = sqrt(-2 ln u1), elements 2p and 2p+1 are
// f32(r cos(2 pi u2) std) and f32(r sin(2 pi u2) std), all in double.
int seeai_plangen_normal(uint64_t seed, uint64_t n, double stddev, float* out) {
  if (!out && n) return 2;
  const uint64_t pairs = (n + 1) / 2;
  constexpr double kInv53 = 1.0 / 9007199254740992.0;
  const double two_pi = 2.0 * M_PI;
  Parallel(pairs, 1 << 16, [&](uint64_t p0, uint64_t p1) {
    for (uint64_t p = p0; p < p1; ++p) {
      const uint64_t x1 = SplitMix(seed, 2 * p + 1), x2 = SplitMix(seed, 2 * p + 2);
      const double u1 = (static_cast<double>(x1 >> 11) + 1.0) * kInv53;
      const double u2 = static_cast<double>(x2 >> 11) * kInv53;
      const double r = std::sqrt(-2.0 * std::log(u1));
      const double a = two_pi * u2;
      out[2 * p] = static_cast<float>(r * std::cos(a) * stddev);
      if (2 * p + 1 < n) out[2 * p + 1] = static_cast<float>(r * std::sin(a) * stddev);
    }
  });
  return 0;
}

// W [rows, cols] row-major: scale[j] = max_i |w[i, j]| / 127 (1 for a zero
// column, at least FLT_MIN); level = clamp(round(w / scale), -127, 127) with
// the quotient in f32 and halves away from zero (arena_binder.cc:129-177).
int seeai_plangen_quantize_cols(const float* w, uint64_t rows, uint64_t cols, int8_t* levels,
                                float* scales) {
  if ((!w || !levels || !scales) && rows * cols) return 2;
  std::vector<float> mx(cols, 0.0f);
  Parallel(cols, 256, [&](uint64_t c0, uint64_t c1) {
    for (uint64_t i = 0; i < rows; ++i)
      for (uint64_t j = c0; j < c1; ++j) mx[j] = std::max(mx[j], std::fabs(w[i * cols + j]));
  });
  for (uint64_t j = 0; j < cols; ++j)
    scales[j] = mx[j] == 0.0f ? 1.0f
                              : std::max(mx[j] / 127.0f, std::numeric_limits<float>::min());
  Parallel(rows, 64, [&](uint64_t r0, uint64_t r1) {
    for (uint64_t i = r0; i < r1; ++i)
      for (uint64_t j = 0; j < cols; ++j) {
        const float q = w[i * cols + j] / scales[j];
        const float r = std::round(q);
        levels[i * cols + j] = static_cast<int8_t>(std::clamp(r, -127.0f, 127.0f));
      }
  });
  return 0;
}

}  // extern "C"
