// Host check of fa::make_fastdiv (fa_internal.h) against plain division; built and run by
// tests/test_fastdiv_cpu.py. Every divisor 1..20000 with edge and random numerators, plus a few
// large divisors. Exits non-zero on the first mismatch.
#include <cstdio>
#include <random>

#include "fa_internal.h"

static uint32_t quotient(uint32_t n, const fa::FastDiv& f) {
  // The kernel's fdiv: __umulhi(n, m) >> s, or n when d == 1.
  return f.d == 1 ? n : static_cast<uint32_t>((static_cast<unsigned long long>(n) * f.m) >> 32) >> f.s;
}

static bool check(uint32_t n, uint32_t d, const fa::FastDiv& f) {
  if (quotient(n, f) == n / d) return true;
  std::printf("mismatch: n=%u d=%u got %u want %u\n", n, d, quotient(n, f), n / d);
  return false;
}

int main() {
  std::mt19937 rng(7);
  long long checks = 0;
  for (uint32_t d = 1; d <= 20000; ++d) {
    const fa::FastDiv f = fa::make_fastdiv(d);
    const uint32_t top = 0x7fffffffu;
    const uint32_t edges[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, top, top - 1,
                              top / d * d, top / d * d - 1};
    for (uint32_t n : edges) {
      if (n > top) continue;
      ++checks;
      if (!check(n, d, f)) return 1;
    }
    for (int i = 0; i < 50; ++i, ++checks) {
      if (!check(rng() & 0x7fffffffu, d, f)) return 1;
    }
  }
  for (uint32_t d : {0x7fffffffu, 0x40000000u, 0x40000001u, 0x3fffffffu, 196608u, 65535u}) {
    const fa::FastDiv f = fa::make_fastdiv(d);
    for (int i = 0; i < 20000; ++i, ++checks) {
      if (!check(rng() & 0x7fffffffu, d, f)) return 1;
    }
  }
  std::printf("fastdiv: %lld checks, all exact\n", checks);
  return 0;
}
