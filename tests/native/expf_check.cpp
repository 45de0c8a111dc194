// Exhaustive check of expf_ref (streamoe_amd/csrc/expf_ref.h) against the
// host libm's expf over every float in [lo, 0] (bit patterns 0x80000000 ..
// 0xC2CFF1B4 = -0x1.9fe368p6, below which both return 0), plus the special
// inputs. Prints "n=<count> mismatches=<count>" and the first mismatches.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "../../streamoe_amd/csrc/expf_ref.h"

static float host_ref(float x) {
  return smoe::expf_ref(x, [](uint32_t i) { return smoe::kExpTab[i]; });
}

int main(int argc, char** argv) {
  const uint32_t lo = 0x80000000u, hi = 0xC2CFF1B4u;
  const uint32_t step = argc > 1 ? (uint32_t)atoi(argv[1]) : 1u;
  const unsigned nt = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 4;
  std::atomic<uint64_t> n{0}, bad{0};
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; ++t)
    th.emplace_back([&, t] {
      uint64_t ln = 0, lb = 0;
      for (uint64_t u = (uint64_t)lo + (uint64_t)t * step; u <= hi; u += (uint64_t)nt * step) {
        float x;
        const uint32_t b = (uint32_t)u;
        memcpy(&x, &b, 4);
        const float a = expf(x), r = host_ref(x);
        ++ln;
        if (memcmp(&a, &r, 4)) {
          if (lb < 3) printf("mismatch x=%a libm=%a ref=%a\n", x, a, r);
          ++lb;
        }
      }
      n += ln;
      bad += lb;
    });
  for (auto& t : th) t.join();
  // Special inputs: the underflow edge and beyond, infinities, NaN, zeros,
  // positive arguments (not produced by a softmax, covered anyway).
  const float sp[] = {-0x1.9fe368p6f, -0x1.9fe36ap6f, -104.0f, -200.0f, -INFINITY, INFINITY, NAN,
                      0.0f, -0.0f, 1e-30f, 1.0f, 10.0f, 88.0f, 88.72f, 89.0f};
  for (float x : sp) {
    const float a = expf(x), r = host_ref(x);
    ++n;
    if (!(memcmp(&a, &r, 4) == 0 || (isnan(a) && isnan(r)))) {
      printf("special mismatch x=%a libm=%a ref=%a\n", x, a, r);
      ++bad;
    }
  }
  printf("n=%llu mismatches=%llu\n", (unsigned long long)n.load(), (unsigned long long)bad.load());
  return bad.load() ? 1 : 0;
}
