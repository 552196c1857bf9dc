// Host check of the single-FMA dequantization predicate (fastpath.hpp).
//
// For every (scale, bias) pair the predicate accepts, the kernels' fast path
// must give the same fp32 value as the dequantization contract fmaf(s, q, b)
// for every quantized value q:
//   4/8-bit low form:  fmaf(s, 1024 + q, c0),       c0 = fmaf(-1024, s, b)
//   4-bit high form:   fmaf(s/16, 1024 + 16 q, c1), c1 = fmaf(-64, s, b)
// Pairs cover every sign and exponent of s and b with a spread of
// significands (bf16 and f16).  Exit status 0 and a summary line on success;
// the first counterexample otherwise.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

// The header under test; the pytest driver points this at altered copies to
// show that the check rejects unsound predicates.
#ifndef CPQ_FASTPATH_HEADER
#define CPQ_FASTPATH_HEADER "../cider_press_amd/csrc/kernels/fastpath.hpp"
#endif
#include CPQ_FASTPATH_HEADER

static float bits_f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

static float bf16_to_f(uint32_t h) { return bits_f(h << 16); }
static float f16_to_f(uint32_t h) {
  const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp((float)(m | 0x400u), (int)e - 25);
  return s ? -v : v;
}

static bool same(float a, float b) { return f_bits(a) == f_bits(b) || (std::isnan(a) && std::isnan(b)); }

struct Stats { long pairs = 0, accepted = 0, checks = 0, quick = 0; };

// Returns false on the first mismatch (printed).
static bool check_pair(const char* tn, uint32_t sv, uint32_t bv, float s, float b, bool full8, Stats& st) {
  const float c0 = std::fmaf(-1024.f, s, b), c1 = std::fmaf(-64.f, s, b);
  const float s16 = s * 0.0625f;
  const int qmax = full8 ? 255 : 15;
  for (int q = 0; q <= qmax; ++q) {
    const float want = std::fmaf(s, (float)q, b);
    const float lo = std::fmaf(s, (float)(1024 + q), c0);
    if (!same(lo, want)) {
      std::printf("MISMATCH %s low form: s=0x%04x b=0x%04x q=%d fast=%a want=%a\n", tn, sv, bv, q, lo, want);
      return false;
    }
    if (q < 16) {
      const float hi = std::fmaf(s16, (float)(1024 + 16 * q), c1);
      if (!same(hi, want)) {
        std::printf("MISMATCH %s high form: s=0x%04x b=0x%04x q=%d fast=%a want=%a\n", tn, sv, bv, q, hi, want);
        return false;
      }
    }
    st.checks++;
  }
  return true;
}

// The packed quick check must imply the exact predicate for each half of a
// word (the other half holds a typical accepted group), and accumulating
// words must keep that property.
template <typename Pred, typename Add, typename Ok>
static bool quick_sound(const char* tn, uint32_t sv, uint32_t bv, uint32_t good_s, uint32_t good_b, Pred pred,
                        Add add, Ok ok, long& quick_accepted) {
  for (int half = 0; half < 2; ++half) {
    cpq::FastQuick a;
    cpq::fast_quick_init(a);
    add(a, good_s | good_s << 16, good_b | good_b << 16);
    const uint32_t s2 = half ? (sv << 16 | good_s) : (good_s << 16 | sv);
    const uint32_t b2 = half ? (bv << 16 | good_b) : (good_b << 16 | bv);
    add(a, s2, b2);
    if (ok(a)) {
      quick_accepted += half == 0;
      if (!pred(sv, bv)) {
        std::printf("MISMATCH %s quick check accepts a rejected pair: s=0x%04x b=0x%04x half=%d\n", tn, sv, bv, half);
        return false;
      }
    }
  }
  return true;
}

template <typename Pred, typename Conv>
static bool sweep(const char* tn, int ebits, int mbits, const std::vector<uint32_t>& mants, Pred pred,
                  Conv conv, Stats& st) {
  std::vector<uint32_t> vals;
  for (uint32_t sign = 0; sign < 2; ++sign)
    for (uint32_t e = 0; e < (1u << ebits); ++e)
      for (uint32_t m : mants) vals.push_back((sign << 15) | (e << mbits) | m);
  for (size_t i = 0; i < vals.size(); ++i) {
    for (size_t j = 0; j < vals.size(); ++j) {
      const uint32_t sv = vals[i], bv = vals[j];
      st.pairs++;
      const bool is_bf16 = ebits == 8;
      const bool q_ok = is_bf16 ? quick_sound(tn, sv, bv, 0x3c24u, 0xbda4u, pred, cpq::fast_quick_add_bf16,
                                              cpq::fast_quick_ok_bf16, st.quick)
                                : quick_sound(tn, sv, bv, 0x211fu, 0xa91fu, pred, cpq::fast_quick_add_f16,
                                              cpq::fast_quick_ok_f16, st.quick);
      if (!q_ok) return false;
      if (!pred(sv, bv)) continue;
      st.accepted++;
      const float s = conv(sv), b = conv(bv);
      if (!std::isfinite(s) || !std::isfinite(b)) {
        std::printf("ACCEPTED NON-FINITE %s s=0x%04x b=0x%04x\n", tn, sv, bv);
        return false;
      }
      if (!check_pair(tn, sv, bv, s, b, ((i * 7 + j) % 13) == 0, st)) return false;
    }
  }
  return true;
}

int main() {
  Stats sb, sf;
  const std::vector<uint32_t> mb = {0x00, 0x01, 0x02, 0x2a, 0x3f, 0x40, 0x41, 0x55, 0x7e, 0x7f};
  const std::vector<uint32_t> mf = {0x000, 0x001, 0x002, 0x155, 0x1ff, 0x200, 0x201, 0x2aa, 0x3fe, 0x3ff};
  if (!sweep("bf16", 8, 7, mb, cpq::fast_ok_bf16, bf16_to_f, sb)) return 1;
  if (!sweep("f16", 5, 10, mf, cpq::fast_ok_f16, f16_to_f, sf)) return 1;
  // Typical quantizations must take the fast path: s ~ U(0.002, 0.02), b = -8 s
  // or -128 s, zero bias, zero group.
  const float ss[] = {0.002f, 0.0037f, 0.01f, 0.019f};
  for (float s : ss) {
    const uint32_t sbf = f_bits(s) >> 16;
    const uint32_t b8 = f_bits(-8.f * bf16_to_f(sbf)) >> 16, b128 = f_bits(-128.f * bf16_to_f(sbf)) >> 16;
    if (!cpq::fast_ok_bf16(sbf, b8) || !cpq::fast_ok_bf16(sbf, b128) || !cpq::fast_ok_bf16(sbf, 0)) {
      std::printf("REJECTED typical bf16 group s=%g\n", s);
      return 1;
    }
  }
  // ... and the packed quick check must take them too (whole words of them).
  {
    cpq::FastQuick a;
    cpq::fast_quick_init(a);
    for (float s : ss) {
      const uint32_t sbf = f_bits(s) >> 16;
      const uint32_t b8 = f_bits(-8.f * bf16_to_f(sbf)) >> 16, b128 = f_bits(-128.f * bf16_to_f(sbf)) >> 16;
      cpq::fast_quick_add_bf16(a, sbf | sbf << 16, b8 | b128 << 16);
    }
    if (!cpq::fast_quick_ok_bf16(a)) {
      std::printf("REJECTED typical bf16 groups by the quick check\n");
      return 1;
    }
    cpq::FastQuick f;
    cpq::fast_quick_init(f);
    cpq::fast_quick_add_f16(f, 0x211f211fu, 0xa91fa91fu);
    cpq::fast_quick_add_f16(f, 0x1c001c00u, 0xa400a000u);  // s = 2^-8, b = -8 s / -2 s
    if (!cpq::fast_quick_ok_f16(f)) {
      std::printf("REJECTED typical f16 groups by the quick check\n");
      return 1;
    }
  }
  if (!cpq::fast_ok_bf16(0, 0) || !cpq::fast_ok_f16(0, 0) || !cpq::fast_ok_f16(0x211f, 0xa91f)) {
    std::printf("REJECTED zero / typical f16 group\n");
    return 1;
  }
  std::printf("ok bf16 pairs=%ld accepted=%ld quick=%ld checks=%ld; f16 pairs=%ld accepted=%ld quick=%ld checks=%ld\n",
              sb.pairs, sb.accepted, sb.quick, sb.checks, sf.pairs, sf.accepted, sf.quick, sf.checks);
  return 0;
}
