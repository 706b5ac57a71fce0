// Compares the device activation math (rustgears_amd/csrc/devmath.h, built
// here for the host) with the host libm over f32 bit patterns
// i = offset + j*stride.  stride 1 covers all 2^32 inputs.
// Usage: devmath_host_check <stride> <offset> <threads>
// Prints one line per function: "<name> <checked> <mismatches> <first_bad_hex>".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../rustgears_amd/csrc/devmath.h"

static float libm_sigmoid(float x) { float e = expf(-x); float d = 1.0f + e; return 1.0f / d; }
static float libm_gelu(float x) {
  float x3 = 0.044715f * x; x3 = x3 * x; x3 = x3 * x;
  float inner = x + x3; float u = 0.7978846f * inner; float t = tanhf(u);
  float h = 0.5f * x; float one_t = 1.0f + t; return h * one_t;
}
static float libm_silu(float x) { float s = libm_sigmoid(x); return x * s; }

struct Count { uint64_t checked = 0, bad = 0; uint32_t first = 0; };
enum { F_TANH, F_EXP, F_SIGMOID, F_GELU, F_SILU, F_TANH_FAST, F_GELU_FAST, NF };
static const char* kNames[NF] = {"tanhf", "expf", "sigmoid", "gelu", "silu", "tanhf_fast", "gelu_fast"};

static bool same(float a, float b) {
  uint32_t x, y; memcpy(&x, &a, 4); memcpy(&y, &b, 4);
  return x == y || (a != a && b != b);
}

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? strtoull(argv[1], 0, 0) : 61;
  const uint64_t offset = argc > 2 ? strtoull(argv[2], 0, 0) : 0;
  const int nt = argc > 3 ? atoi(argv[3]) : 8;
  std::vector<std::vector<Count>> res(nt, std::vector<Count>(NF));
  std::vector<std::thread> th;
  for (int t = 0; t < nt; t++)
    th.emplace_back([&, t] {
      for (uint64_t i = offset + (uint64_t)t * stride; i < (1ull << 32); i += (uint64_t)nt * stride) {
        const float x = rgmath::bitsf((uint32_t)i);
        const float got[NF] = {rgmath::tanhf_fdlibm(x), rgmath::expf_aor(x), rgmath::sigmoid(x), rgmath::gelu(x),
                               rgmath::act_apply(rgmath::ACT_SILU, 0.0f, x), rgmath::tanhf_fast(x),
                               rgmath::gelu_fast(x)};
        const float want[NF] = {tanhf(x), expf(x), libm_sigmoid(x), libm_gelu(x), libm_silu(x), tanhf(x),
                                libm_gelu(x)};
        for (int f = 0; f < NF; f++) {
          Count& c = res[t][f];
          c.checked++;
          if (!same(got[f], want[f])) { if (!c.bad) c.first = (uint32_t)i; c.bad++; }
        }
      }
    });
  for (auto& x : th) x.join();
  for (int f = 0; f < NF; f++) {
    Count tot;
    for (int t = 0; t < nt; t++) {
      tot.checked += res[t][f].checked;
      if (res[t][f].bad && !tot.bad) tot.first = res[t][f].first;
      tot.bad += res[t][f].bad;
    }
    printf("%s %llu %llu %08x\n", kNames[f], (unsigned long long)tot.checked, (unsigned long long)tot.bad, tot.first);
  }
  return 0;
}
