// Exhaustive host check of the gfx950 kernels' nearest-code searches, the
// binary one and the bucketed one (vkqlora.rs_amd/csrc/qh_nf4.h), against the oracle's 16-level scan
// (oracle/qlora_oracle.c, quant.rs:263-278), for every float in [-1, 1]
// (the range of fl(w/absmax) for finite w) plus special values.
// Prints "mismatches=<n> checked=<n>".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "qh_nf4.h"
#include "qlora_oracle.h"

static float f_of(uint32_t b) {
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

static uint32_t bucketed(float t) {
  static constexpr QhNf4Buckets B = qh_nf4_make_buckets();
  const uint32_t c0 = B.c0[qh_nf4_bucket(t)];
  return qh_nf4_code_bucketed(t, c0, qh_nf4_levels[c0], qh_nf4_levels[c0 + 1],
                              qh_nf4_levels[c0 + 2]);
}

int main() {
  static const float L[17] = QH_NF4_LUT17_INIT;
  for (int j = 0; j < 17; ++j)
    if (std::memcmp(&L[j], &qh_nf4_levels[j], 4) != 0) {
      std::printf("level table mismatch at %d\n", j);
      return 1;
    }
  long long bad = 0, checked = 0;
  const uint32_t top = 0x3F800000u;  // 1.0f
#pragma omp parallel for reduction(+ : bad, checked) schedule(static)
  for (long long i = 0; i <= (long long)top; ++i) {
    for (int sgn = 0; sgn < 2; ++sgn) {
      float t = f_of((uint32_t)i | (sgn ? 0x80000000u : 0u));
      uint32_t fast = qh_nf4_code_of_target(t, L);
      uint32_t ref = or_nearest_nf4_code(t, 1.0f);
      bad += fast != ref;
      bad += bucketed(t) != ref;
      checked += 2;
    }
  }
  const float specials[] = {NAN, -NAN, INFINITY, -INFINITY, 1.5f, -1.5f, 1e30f,
                            -1e30f, 0.0f, -0.0f, 1e-45f, -1e-45f};
  for (float t : specials) {
    bad += qh_nf4_code_of_target(t, L) != or_nearest_nf4_code(t, 1.0f);
    ++checked;
  }
  // the bucketed search serves |t| <= 1 and NaN (a quotient w / absmax)
  const float nans[] = {NAN, -NAN, f_of(0x7FC00001u), f_of(0xFFBFFFFFu), f_of(0x7F800001u)};
  for (float t : nans) {
    bad += bucketed(t) != or_nearest_nf4_code(t, 1.0f);
    ++checked;
  }
  std::printf("mismatches=%lld checked=%lld\n", bad, checked);
  return bad != 0;
}
