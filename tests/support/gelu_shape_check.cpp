// Exhaustive host check of two properties of the exact GELU (rgmath::gelu:
// the reference's f32 roundings over glibc tanhf, equal to glibc on every
// input) that the INT8 GELU requantization relies on to take a per-tensor
// absmax from the largest pre-activation:
//   1. on [0, +inf] the f32 GELU never decreases: gelu(next(x)) >= gelu(x)
//      for every pair of consecutive non-negative f32 values;
//   2. over every negative f32 (finite or -inf) |gelu(x)| is at most
//      rgmath::kGeluNegAbsMax (NaN results, which the absmax ignores, are
//      skipped), and that bound is attained.
//   3. (the certified FP16 hand-off) fp16_bits(round_fp16(y)) is monotonic
//      in y over the finite f32 values and never gives -0.
// Prints "monotone <checked> <violations> <first_bad_hex>",
// "negmax <checked> <max_bits_hex> <argmax_hex> <exceeds_bound>" and
// "fp16mono <checked pairs> <violations> <first_bad_hex>".
// Usage: gelu_shape_check <threads> [stride]: with stride s > 1 only every
// s-th block of 2^16 consecutive bit patterns is walked (all of them at 1).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

#include "../../rustgears_amd/csrc/devmath.h"

int main(int argc, char** argv) {
  const int nt = argc > 1 ? atoi(argv[1]) : 8;
  const uint64_t stride = argc > 2 ? strtoull(argv[2], 0, 0) : 1;
  const uint64_t kBlock = 1u << 16;
  auto walked = [&](uint64_t i) { return (i / kBlock) % stride == 0; };
  // 1. non-negative values: bits 0 .. 0x7f800000 (+inf) in increasing order
  const uint32_t last = 0x7f800000u;
  std::vector<uint64_t> checked(nt), bad(nt);
  std::vector<uint32_t> first(nt, 0xffffffffu);
  std::vector<std::thread> th;
  for (int w = 0; w < nt; w++)
    th.emplace_back([&, w] {
      const uint64_t lo = (uint64_t)last * w / nt, hi = (uint64_t)last * (w + 1) / nt;  // pairs (i, i+1), i in [lo, hi)
      float prev = rgmath::gelu(rgmath::bitsf((uint32_t)lo));
      for (uint64_t i = lo; i < hi; i++) {
        if (!walked(i)) {
          i = (i / kBlock + 1) * kBlock - 1;  // skip to the block's last value: the next walked pair starts fresh
          if (i + 1 < hi) prev = rgmath::gelu(rgmath::bitsf((uint32_t)(i + 1)));
          continue;
        }
        const float next = rgmath::gelu(rgmath::bitsf((uint32_t)(i + 1)));
        checked[w]++;
        if (!(next >= prev) && bad[w]++ == 0) first[w] = (uint32_t)i;
        prev = next;
      }
    });
  for (auto& t : th) t.join();
  uint64_t c = 0, b = 0;
  uint32_t f = 0xffffffffu;
  for (int w = 0; w < nt; w++) {
    c += checked[w];
    b += bad[w];
    if (first[w] < f) f = first[w];
  }
  printf("monotone %llu %llu %08x\n", (unsigned long long)c, (unsigned long long)b, f);

  // 2. negative values: bits 0x80000000 .. 0xff800000 (-0 .. -inf)
  th.clear();
  std::vector<uint32_t> mx(nt, 0), arg(nt, 0);
  std::vector<uint64_t> nchk(nt, 0);
  const uint64_t nlo = 0x80000000ull, nhi = 0xff800001ull;
  for (int w = 0; w < nt; w++)
    th.emplace_back([&, w] {
      const uint64_t lo = nlo + (nhi - nlo) * w / nt, hi = nlo + (nhi - nlo) * (w + 1) / nt;
      for (uint64_t i = lo; i < hi; i++) {
        if (!walked(i) && i != 0xbf409c70u) continue;  // the sampled walk still visits the argmax
        const float g = rgmath::gelu(rgmath::bitsf((uint32_t)i));
        nchk[w]++;
        if (g != g) continue;
        const uint32_t a = rgmath::fbits(g) & 0x7fffffffu;
        if (a > mx[w]) { mx[w] = a; arg[w] = (uint32_t)i; }
      }
    });
  for (auto& t : th) t.join();
  uint32_t m = 0, am = 0;
  uint64_t nc = 0;
  for (int w = 0; w < nt; w++) {
    nc += nchk[w];
    if (mx[w] > m) { m = mx[w]; am = arg[w]; }
  }
  printf("negmax %llu %08x %08x %d\n", (unsigned long long)nc, m, am,
         (int)(m > rgmath::fbits(rgmath::kGeluNegAbsMax)));

  // 3. the FP16 operand of a value, h(y) = fp16_bits(round_fp16(y)), never
  // decreases (as the binary16 value it encodes) over the finite f32 values
  // in increasing order, and is never -0: equal h at both ends of an interval
  // then means equal h inside it.  Walk: bits 0xff7fffff (-max) down to
  // 0x80000000 (-0), then 0 up to 0x7f7fffff (+max), as one sequence of
  // 2^32 - 2^24 - 1 steps (-0 and +0 are one value).
  auto h_key = [](float y) -> int32_t {
    const uint16_t h = rgmath::fp16_bits(rgmath::round_fp16(y));
    return (h & 0x8000u) ? -(int32_t)(h & 0x7fffu) - (h == 0x8000u ? 1 << 20 : 0) : (int32_t)h;  // -0 fails
  };
  auto seq = [](uint64_t k) -> uint32_t {  // k-th finite f32 in increasing order
    const uint64_t nneg = 0xff7fffffull - 0x80000000ull + 1;  // -max .. -0
    return k < nneg ? (uint32_t)(0xff7fffffull - k) : (uint32_t)(k - nneg + 1);  // then +min .. +max (skip +0)
  };
  const uint64_t total = (0xff7fffffull - 0x80000000ull + 1) + 0x7f7fffffull;
  th.clear();
  std::vector<uint64_t> hchk(nt, 0), hbad(nt, 0);
  std::vector<uint32_t> hfirst(nt, 0xffffffffu);
  for (int w = 0; w < nt; w++)
    th.emplace_back([&, w] {
      const uint64_t lo = (total - 1) * w / nt, hi = (total - 1) * (w + 1) / nt;  // pairs (k, k+1)
      int32_t prev = h_key(rgmath::bitsf(seq(lo)));
      for (uint64_t k = lo; k < hi; k++) {
        if (!walked(k)) {
          k = (k / kBlock + 1) * kBlock - 1;
          if (k + 1 < hi) prev = h_key(rgmath::bitsf(seq(k + 1)));
          continue;
        }
        const int32_t next = h_key(rgmath::bitsf(seq(k + 1)));
        hchk[w]++;
        if (!(next >= prev) && hbad[w]++ == 0) hfirst[w] = seq(k);
        prev = next;
      }
    });
  for (auto& t : th) t.join();
  uint64_t hc = 0, hb = 0;
  uint32_t hf = 0xffffffffu;
  for (int w = 0; w < nt; w++) {
    hc += hchk[w];
    hb += hbad[w];
    if (hfirst[w] < hf) hf = hfirst[w];
  }
  printf("fp16mono %llu %llu %08x\n", (unsigned long long)hc, (unsigned long long)hb, hf);
  return 0;
}
