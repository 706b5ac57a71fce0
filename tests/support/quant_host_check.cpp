// Compares rgmath::quantize_rz (the fused requantization's quantizer, built
// here for the host) with the reference rule of QuantTensor::from_f32
// (quantize.rs:22: round half away from zero, clamp to +-127, `as i8`, NaN
// -> 0) over f32 bit patterns t = offset + j*stride; stride 1 covers all
// 2^32 inputs.  Usage: quant_host_check <stride> <offset> <threads> [bound]
// Prints "<checked> <mismatches> <first_bad_hex>".
// With "bound", the bit patterns are absmax values instead: for every finite
// absmax >= 0 the largest quantized magnitude t = absmax * inv (inv = 1 /
// scale_from_absmax(absmax), rounding is monotonic, so |v| <= absmax gives
// |v * inv| <= t) must stay below 127.5 and quantize_rz_bounded(t) must
// equal quantize_rz(t).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../rustgears_amd/csrc/devmath.h"

static int32_t reference(float t) {
  float r = roundf(t);
  if (r < -127.0f) r = -127.0f;
  if (r > 127.0f) r = 127.0f;
  if (r != r) return 0;
  return (int32_t)r;
}

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? strtoull(argv[1], 0, 0) : 61;
  const uint64_t offset = argc > 2 ? strtoull(argv[2], 0, 0) : 0;
  const int nt = argc > 3 ? atoi(argv[3]) : 8;
  const bool bound = argc > 4 && strcmp(argv[4], "bound") == 0;
  std::vector<uint64_t> checked(nt), bad(nt);
  std::vector<uint32_t> first(nt, 0);
  std::vector<std::thread> th;
  const uint64_t total = ((1ull << 32) - offset + stride - 1) / stride;
  for (int w = 0; w < nt; w++)
    th.emplace_back([&, w] {
      for (uint64_t j = w; j < total; j += nt) {
        const uint32_t bits = (uint32_t)(offset + j * stride);
        float t;
        memcpy(&t, &bits, 4);
        if (bound) {
          if (bits >= 0x7f800000u) continue;  // negative, inf and NaN absmax values do not occur
          const float inv = 1.0f / rgmath::scale_from_absmax(t);
          const float q = t * inv;
          checked[w]++;
          if ((!(fabsf(q) < 127.5f) || rgmath::quantize_rz_bounded(q) != rgmath::quantize_rz(q) ||
               rgmath::quantize_rz_bounded(-q) != rgmath::quantize_rz(-q)) &&
              bad[w]++ == 0)
            first[w] = bits;
          continue;
        }
        checked[w]++;
        if (rgmath::quantize_rz(t) != reference(t) && bad[w]++ == 0) first[w] = bits;
      }
    });
  for (auto& x : th) x.join();
  uint64_t c = 0, b = 0;
  uint32_t f = 0;
  for (int w = 0; w < nt; w++) {
    c += checked[w];
    if (bad[w] && !b) f = first[w];
    b += bad[w];
  }
  printf("%llu %llu %08x\n", (unsigned long long)c, (unsigned long long)b, f);
  return 0;
}
