// qh_nf4.h -- NF4 codebook and the exact nearest-code search, shared by the
// gfx950 kernels and the host-side exhaustive check of the search.
//
// The codebook is qlora-core/src/quant.rs:27-44 (ascending; every f64
// literal there is exactly representable in f32).  The nearest-code rule
// is quant.rs:263-278: the FIRST j minimising fl(|L_j - t|), t = fl(w/absmax),
// with code 7 for an all-zero block.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define QH_HD __host__ __device__
#else
#define QH_HD
#endif

// 16 levels followed by a +inf sentinel so that L[c+1] is always readable.
#define QH_NF4_LUT17_INIT                                                    \
  {-1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, \
   -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f, \
   0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,         \
   0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,          \
   0.7229568362236023f, 1.0f, __builtin_inff()}

#define QH_NF4_ZERO_CODE 7u
#define QH_DQ_BLOCK 256

// Nearest code for a target t = fl(w/absmax), given the 17-entry table.
//
// fl(x) is monotone, so for levels below t the distance fl(t - L_j) is
// non-increasing in j and for levels above t the distance fl(L_j - t) is
// non-decreasing.  The minimum is therefore at c = max{j : L_j <= t} or at
// c + 1; on a tie the reference keeps the first index (strict `<`), i.e. c.
// Distinct levels are >= 0.0795 apart while |t - L_j| <= 2, so no two
// distances on one side can round to the same value: the first minimum is
// one of c, c+1.  NaN targets fail every comparison and give code 0, as the
// reference's scan does.  The host test checks this against the scan for
// every float in [-1, 1] and the special values.
// Targets with |t| > 1 cannot come from w / absmax (|w| <= absmax); for them
// the distances may round together, so the plain scan is used.
QH_HD inline uint32_t qh_nf4_code_of_target(float t, const float *L) {
  if (__builtin_fabsf(t) > 1.0f) {
    uint32_t best = 0;
    float bd = __builtin_inff();
    for (uint32_t j = 0; j < 16; ++j) {
      float d = __builtin_fabsf(L[j] - t);
      if (d < bd) {
        bd = d;
        best = j;
      }
    }
    return best;
  }
  uint32_t c = (t >= L[8]) ? 8u : 0u;
  c += (t >= L[c + 4]) ? 4u : 0u;
  c += (t >= L[c + 2]) ? 2u : 0u;
  c += (t >= L[c + 1]) ? 1u : 0u;
  float lo = L[c], hi = L[c + 1];
  float d0 = __builtin_fabsf(lo - t);
  float d1 = __builtin_fabsf(hi - t);
  return (d1 < d0) ? c + 1u : c;
}

// ---- bucketed search: one table read and one comparison per target ------
// A target's bucket is its float bits >> 20: sign, exponent and the top
// three mantissa bits (4096 buckets).  Inside [-1, 1] a bucket spans at most
// an eighth of an octave (<= 1/16 wide), less than the gap between any two
// adjacent levels (>= 0.0795), so c(t) = max{j : L_j <= t} takes at most two
// values on it: c0 = c(the bucket's lowest target) and c0 + 1.  Buckets of
// exponent 255 (inf, NaN) get c0 = 0.  The host test checks the bucketed
// search against the scan for every float in [-1, 1].
#define QH_NF4_BUCKETS 4096

constexpr float qh_nf4_levels[18] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f, __builtin_inff(), __builtin_inff()};

constexpr uint32_t qh_nf4_floor_code(float t) {
  uint32_t c = 0;
  for (uint32_t j = 1; j < 16; ++j)
    if (qh_nf4_levels[j] <= t) c = j;
  return c;
}

// 16-byte aligned: the kernels copy it to LDS with 16-byte loads
struct alignas(16) QhNf4Buckets {
  uint8_t c0[QH_NF4_BUCKETS];
};

constexpr QhNf4Buckets qh_nf4_make_buckets() {
  QhNf4Buckets b{};
  for (uint32_t i = 0; i < QH_NF4_BUCKETS; ++i) {
    // the lowest target: the bucket's smallest magnitude when positive, its
    // largest when negative
    const uint32_t bits = (i >> 11) ? ((i << 20) | 0xFFFFFu) : (i << 20);
    const bool special = ((i >> 3) & 0xFFu) == 0xFFu;
    b.c0[i] = special ? 0 : (uint8_t)qh_nf4_floor_code(__builtin_bit_cast(float, bits));
  }
  return b;
}

QH_HD inline uint32_t qh_nf4_bucket(float t) { return __builtin_bit_cast(uint32_t, t) >> 20; }

// The nearest code of a target |t| <= 1 (or NaN) from its bucket's c0 and the
// levels L[c0], L[c0 + 1], L[c0 + 2] (+inf past L[15]): c = c0 + (t >= L[c0+1]),
// then c or c + 1 by the rule of qh_nf4_code_of_target (ties keep c).  NaN
// fails every comparison: c0 = 0 and code 0.
QH_HD inline uint32_t qh_nf4_code_bucketed(float t, uint32_t c0, float l0, float l1, float l2) {
  const bool up = t >= l1;
  const float lo = up ? l1 : l0, hi = up ? l2 : l1;
  const float d0 = __builtin_fabsf(lo - t), d1 = __builtin_fabsf(hi - t);
  return c0 + (up ? 1u : 0u) + (d1 < d0 ? 1u : 0u);
}

// Rust `(x).round() as i32` followed by `.clamp(-127, 127)`: round half
// away from zero, saturating cast with NaN -> 0 (quant.rs:293,
// optim.rs:91).
QH_HD inline int32_t qh_round_clamp127(float x) {
  if (x != x) return 0;
  float r = __builtin_roundf(x);
  if (r > 127.0f) return 127;
  if (r < -127.0f) return -127;
  return (int32_t)r;
}
