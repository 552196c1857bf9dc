// When the single-FMA dequantization is exact (host and device).
//
// The fast path computes w = fmaf(s, 1024 + q, c0) with c0 = b - 1024*s (and,
// for a nibble left in the high half of a byte, fmaf(s/16, 1024 + 16q, c1)
// with c1 = b - 64*s).  s*(1024+q) is exact inside the FMA, so the result is
// RN(s*q + b) == fmaf(s, q, b) exactly when c0 and c1 are exact fp32 values
// and s/16 is not subnormal.  These predicates decide that from the raw
// 16-bit patterns of s and b with integer compares only (no branches, so a
// workgroup can check hundreds of groups in a few instructions).
//
// bf16 (bias 127, 8-bit significand): d = e(b) - e(s) must lie in [-5, 21]
// (|d - 10| <= 15 and |d - 6| <= 15 keep b - 1024 s and b - 64 s inside 24
// significant bits), e(s) in [27, 240] and e(b) in [27, 253] (|b| < 2^127,
// so c0 = b - 1024 s stays finite).  f16 (bias 15, 11-bit
// significand): d in [-2, 18]; s must be normal.  A zero s or b is fine
// (then c0, c1 are b or -1024 s / -64 s) except for the sign of a zero
// result: with b = -0 and a negative (or -0) s, fmaf(s, 0, b) is -0 while
// the fast path's exact cancellation gives +0, so that pair is rejected.
// A non-finite b is never accepted.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define CPQ_HD __host__ __device__ __forceinline__
#else
#define CPQ_HD inline
#endif

namespace cpq {

CPQ_HD bool fast_ok_bf16(uint32_t sv, uint32_t bv) {
  const uint32_t es = (sv >> 7) & 0xffu, eb = (bv >> 7) & 0xffu;
  const bool sz = (sv & 0x7fffu) == 0u, bz = (bv & 0x7fffu) == 0u;
  const bool b_norm = eb - 27u < 227u;     // 27 <= e(b) <= 253: b - 1024 s cannot overflow
  const bool s_rng = es - 27u <= 213u;     // 27 <= e(s) <= 240
  const bool d_ok = eb - es + 5u <= 26u;   // -5 <= e(b) - e(s) <= 21
  const bool z_ok = !((bv == 0x8000u) & ((sv & 0x8000u) != 0u));  // see zero signs above
  return z_ok & ((sz & (bz | b_norm)) | (!sz & s_rng & (bz | (b_norm & d_ok))));
}

CPQ_HD bool fast_ok_f16(uint32_t sv, uint32_t bv) {
  const uint32_t es = (sv >> 10) & 0x1fu, eb = (bv >> 10) & 0x1fu;
  const bool sz = (sv & 0x7fffu) == 0u, bz = (bv & 0x7fffu) == 0u;
  const bool b_norm = eb - 1u < 30u;       // 1 <= e(b) < 31
  const bool s_rng = es - 1u < 30u;        // s normal
  const bool d_ok = eb - es + 2u <= 20u;   // -2 <= e(b) - e(s) <= 18
  const bool z_ok = !((bv == 0x8000u) & ((sv & 0x8000u) != 0u));
  return z_ok & ((sz & (bz | b_norm)) | (!sz & s_rng & (bz | (b_norm & d_ok))));
}

// Packed sufficient check for many groups at once.  Each 32-bit word holds
// two 16-bit scales (or biases); per 16-bit half it tracks three running
// maxima of biased exponent fields (exponent kept in place, so one AND per
// word), with unsigned 16-bit wrap-around turning "below range" into "large":
//   e(s) - lo,  e(b) - lo,  e(b) - e(s) + dlo.
// All maxima within their limits means every group seen is normal, in range
// and within the exponent gap -- a subset of what fast_ok_* accepts (zero
// scales or biases fall outside it and are left to the exact predicate).
typedef uint16_t u16x2_t __attribute__((vector_size(4)));

struct FastQuick {
  u16x2_t m1, m2, m3;
};

CPQ_HD u16x2_t u16x2_of(uint32_t v) {
  u16x2_t r;
  __builtin_memcpy(&r, &v, 4);
  return r;
}

CPQ_HD u16x2_t u16x2_max(u16x2_t a, u16x2_t b) {
#if defined(__clang__)
  return __builtin_elementwise_max(a, b);
#else
  u16x2_t r;
  r[0] = a[0] > b[0] ? a[0] : b[0];
  r[1] = a[1] > b[1] ? a[1] : b[1];
  return r;
#endif
}

CPQ_HD void fast_quick_init(FastQuick& a) {
  a.m1 = u16x2_of(0u);
  a.m2 = u16x2_of(0u);
  a.m3 = u16x2_of(0u);
}

template <uint32_t MASK, uint32_t LO, uint32_t DLO>
CPQ_HD void fast_quick_add_t(FastQuick& a, uint32_t s2, uint32_t b2) {
  const u16x2_t es = u16x2_of(s2 & (MASK | MASK << 16)), eb = u16x2_of(b2 & (MASK | MASK << 16));
  const u16x2_t lo = u16x2_of(LO | LO << 16), dlo = u16x2_of(DLO | DLO << 16);
  a.m1 = u16x2_max(a.m1, es - lo);
  a.m2 = u16x2_max(a.m2, eb - lo);
  a.m3 = u16x2_max(a.m3, eb - es + dlo);
}

template <uint32_t L1, uint32_t L2, uint32_t L3>
CPQ_HD bool fast_quick_ok_t(const FastQuick& a) {
  return (a.m1[0] <= L1) & (a.m1[1] <= L1) & (a.m2[0] <= L2) & (a.m2[1] <= L2) & (a.m3[0] <= L3) &
         (a.m3[1] <= L3);
}

// bf16: exponent field 0x7f80 (e << 7); e(s) in [27, 240], e(b) in [27, 253],
// e(b) - e(s) in [-5, 21].
CPQ_HD void fast_quick_add_bf16(FastQuick& a, uint32_t s2, uint32_t b2) {
  fast_quick_add_t<0x7f80u, 27u << 7, 5u << 7>(a, s2, b2);
}
CPQ_HD bool fast_quick_ok_bf16(const FastQuick& a) {
  return fast_quick_ok_t<(240u - 27u) << 7, (253u - 27u) << 7, 26u << 7>(a);
}

// f16: exponent field 0x7c00 (e << 10); e(s), e(b) in [1, 30], e(b) - e(s) in [-2, 18].
CPQ_HD void fast_quick_add_f16(FastQuick& a, uint32_t s2, uint32_t b2) {
  fast_quick_add_t<0x7c00u, 1u << 10, 2u << 10>(a, s2, b2);
}
CPQ_HD bool fast_quick_ok_f16(const FastQuick& a) {
  return fast_quick_ok_t<29u << 10, 29u << 10, 20u << 10>(a);
}

}  // namespace cpq
