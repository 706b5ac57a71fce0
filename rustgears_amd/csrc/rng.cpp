// rng.cpp — the reference's SplitMix64 generator (src/rng.rs:10-98) for
// building its seeded weights and inputs: Rng::new xors the seed with the
// golden gamma (rng.rs:16-18), next_u64 is SplitMix64 (21-27), uniform takes
// the top 24 bits (30-32), uniform_range is lo + (hi-lo)*u (35-37) and normal
// is Box-Muller with u1 clamped to 1e-7 (40-44).  The global generator starts
// from seed 0x5EED (rng.rs:66) and manual_seed replaces it (71-73).
// Compiled with -ffp-contract=off; logf/cosf are the host libm, as in Rust.
#include <cmath>
#include <cstdint>
#include <mutex>

#include "../../include/rgnpu.h"

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

struct SplitMix {
  uint64_t state;
  explicit SplitMix(uint64_t seed) : state(seed ^ kGamma) {}
  uint64_t next() {
    state += kGamma;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  float uniform() { return (float)(next() >> 40) / (float)(1ull << 24); }
  float uniform_range(float lo, float hi) {
    const float span = hi - lo;
    const float u = uniform();
    const float scaled = span * u;
    return lo + scaled;
  }
  float normal() {
    float u1 = uniform();
    u1 = std::fmax(u1, 1e-7f);
    const float u2 = uniform();
    const float radius = std::sqrt(-2.0f * std::log(u1));
    const float angle = (2.0f * 3.14159274101257324f) * u2;
    return radius * std::cos(angle);
  }
};

std::mutex g_mu;
SplitMix g_rng(0x5EEDull);

}  // namespace

extern "C" {

void rgnpu_manual_seed(uint64_t seed) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_rng = SplitMix(seed);
}

void rgnpu_fill_uniform(float* out, int64_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (int64_t i = 0; i < n; i++) out[i] = g_rng.uniform();
}

void rgnpu_fill_uniform_range(float* out, int64_t n, float lo, float hi) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (int64_t i = 0; i < n; i++) out[i] = g_rng.uniform_range(lo, hi);
}

void rgnpu_fill_normal(float* out, int64_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (int64_t i = 0; i < n; i++) out[i] = g_rng.normal();
}

}  // extern "C"
