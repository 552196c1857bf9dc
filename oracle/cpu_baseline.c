/* CPU baseline of the quantized matmul: dequantize-and-dot on the host.
 *
 * TEST AND MEASUREMENT INFRASTRUCTURE ONLY: loaded by tests/ and by the
 * cpu_baseline leg of bench.py, never by the product library.
 *
 * Semantics are the GPU path's (and the reference's, quantized.h:2589-2600
 * for the packing, qmv_dispatch_bench.rs:37-43 for the byte count the
 * benchmark divides by): each weight is dequantized to T as
 * RNE_T(fmaf(scale, q, bias)), products of the T-rounded weight and the
 * activation accumulate in fp32, and the sum is rounded to T once.  The
 * summation order differs between forms (lane-wise partial sums), so forms
 * agree with each other and the oracle to the matmul tolerance, not bit for
 * bit.  Finite inputs only (the rounding helpers do not special-case NaN).
 *
 * Three forms, each a complete kernel, chosen at run time:
 *   scalar  -- plain C, built without auto-vectorisation;
 *   avx2    -- 8 weights per step (AVX2 + FMA + F16C);
 *   avx512  -- 16 weights per step (AVX-512 F/BW/VL).
 * The SIMD forms handle 4-bit weights with group sizes that are multiples
 * of 16; other widths fall back to the scalar form.  Work is split over N
 * rows between `threads` pthreads; each thread dequantizes one weight row
 * into fp32 once and dots it with every activation row. */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { CB_F16 = 1, CB_BF16 = 2 };
enum { CB_SCALAR = 0, CB_AVX2 = 1, CB_AVX512 = 2 };

/* ---- scalar conversions (round to nearest even) ---- */
static inline float cb_bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t cb_f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float cb_to_f32(uint16_t h, int dtype) {
  if (dtype == CB_BF16) return cb_bits_to_f32((uint32_t)h << 16);
  return _cvtsh_ss(h);
}
static inline uint16_t cb_from_f32(float f, int dtype) {
  if (dtype == CB_BF16) {
    uint32_t u = cb_f32_bits(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
  return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}
static inline float cb_round_t(float f, int dtype) { return cb_to_f32(cb_from_f32(f, dtype), dtype); }

typedef struct {
  const uint16_t* x;
  size_t m;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  size_t n0, n1, n, k;
  int gs, bits, dtype, form;
  uint16_t* y;
} cb_job;

/* ---- scalar form ---- */
__attribute__((optimize("no-tree-vectorize"))) static void cb_row_scalar(const cb_job* j, size_t r, float* wrow) {
  const size_t k = j->k, wpr = k * (size_t)j->bits / 32u, gpr = k / (size_t)j->gs;
  const uint32_t* wr = j->w + r * wpr;
  const uint32_t mask = (1u << j->bits) - 1u;
  for (size_t g = 0; g < gpr; ++g) {
    const float s = cb_to_f32(j->s[r * gpr + g], j->dtype), b = cb_to_f32(j->b[r * gpr + g], j->dtype);
    for (size_t i = g * (size_t)j->gs; i < (g + 1) * (size_t)j->gs; ++i) {
      const size_t bit = i * (size_t)j->bits, wi = bit / 32u, sh = bit % 32u;
      uint64_t v = wr[wi];
      if (sh + (size_t)j->bits > 32u) v |= (uint64_t)wr[wi + 1] << 32;
      const uint32_t q = (uint32_t)(v >> sh) & mask;
      wrow[i] = cb_round_t(fmaf(s, (float)q, b), j->dtype);
    }
  }
}

__attribute__((optimize("no-tree-vectorize"))) static float cb_dot_scalar(const float* a, const float* b, size_t k) {
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  size_t i = 0;
  for (; i + 4 <= k; i += 4)
    for (int l = 0; l < 4; ++l) acc[l] += a[i + l] * b[i + l];
  float t = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  for (; i < k; ++i) t += a[i] * b[i];
  return t;
}

/* ---- AVX2 form (4-bit) ---- */
__attribute__((target("avx2,fma,f16c"))) static inline __m256 cb_round_t8(__m256 v, int dtype) {
  if (dtype == CB_BF16) {
    __m256i u = _mm256_castps_si256(v);
    __m256i lsb = _mm256_and_si256(_mm256_srli_epi32(u, 16), _mm256_set1_epi32(1));
    u = _mm256_add_epi32(u, _mm256_add_epi32(lsb, _mm256_set1_epi32(0x7FFF)));
    return _mm256_castsi256_ps(_mm256_and_si256(u, _mm256_set1_epi32((int)0xFFFF0000u)));
  }
  return _mm256_cvtph_ps(_mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
}

__attribute__((target("avx2,fma,f16c"))) static void cb_row_avx2(const cb_job* j, size_t r, float* wrow) {
  const size_t k = j->k, wpr = k / 8u, gpr = k / (size_t)j->gs;
  const uint32_t* wr = j->w + r * wpr;
  const __m256i shifts = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
  const __m256i lo4 = _mm256_set1_epi32(15);
  for (size_t g = 0; g < gpr; ++g) {
    const __m256 s = _mm256_set1_ps(cb_to_f32(j->s[r * gpr + g], j->dtype));
    const __m256 b = _mm256_set1_ps(cb_to_f32(j->b[r * gpr + g], j->dtype));
    for (size_t i = g * (size_t)j->gs; i < (g + 1) * (size_t)j->gs; i += 8) {
      const __m256i word = _mm256_set1_epi32((int)wr[i / 8]);
      const __m256 q = _mm256_cvtepi32_ps(_mm256_and_si256(_mm256_srlv_epi32(word, shifts), lo4));
      _mm256_storeu_ps(wrow + i, cb_round_t8(_mm256_fmadd_ps(s, q, b), j->dtype));
    }
  }
}

__attribute__((target("avx2,fma"))) static float cb_dot_avx2(const float* a, const float* b, size_t k) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  size_t i = 0;
  for (; i + 16 <= k; i += 16) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), acc1);
  }
  __m256 acc = _mm256_add_ps(acc0, acc1);
  __m128 h = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
  h = _mm_add_ps(h, _mm_movehl_ps(h, h));
  h = _mm_add_ss(h, _mm_movehdup_ps(h));
  float t = _mm_cvtss_f32(h);
  for (; i < k; ++i) t += a[i] * b[i];
  return t;
}

/* ---- AVX-512 form (4-bit) ---- */
__attribute__((target("avx512f,avx512bw,avx512vl"))) static inline __m512 cb_round_t16(__m512 v, int dtype) {
  if (dtype == CB_BF16) {
    __m512i u = _mm512_castps_si512(v);
    __m512i lsb = _mm512_and_si512(_mm512_srli_epi32(u, 16), _mm512_set1_epi32(1));
    u = _mm512_add_epi32(u, _mm512_add_epi32(lsb, _mm512_set1_epi32(0x7FFF)));
    return _mm512_castsi512_ps(_mm512_and_si512(u, _mm512_set1_epi32((int)0xFFFF0000u)));
  }
  return _mm512_cvtph_ps(_mm512_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
}

__attribute__((target("avx512f,avx512bw,avx512vl"))) static void cb_row_avx512(const cb_job* j, size_t r,
                                                                              float* wrow) {
  const size_t k = j->k, wpr = k / 8u, gpr = k / (size_t)j->gs;
  const uint32_t* wr = j->w + r * wpr;
  const __m128i nib = _mm_set1_epi8(15);
  for (size_t g = 0; g < gpr; ++g) {
    const __m512 s = _mm512_set1_ps(cb_to_f32(j->s[r * gpr + g], j->dtype));
    const __m512 b = _mm512_set1_ps(cb_to_f32(j->b[r * gpr + g], j->dtype));
    for (size_t i = g * (size_t)j->gs; i < (g + 1) * (size_t)j->gs; i += 16) {
      /* 16 nibbles (8 bytes): low nibbles are the even elements, high nibbles
       * the odd ones; interleaving the two byte vectors restores k order. */
      uint64_t v;
      memcpy(&v, wr + i / 8, 8);
      const __m128i bytes = _mm_cvtsi64_si128((long long)v);
      const __m128i lo = _mm_and_si128(bytes, nib), hi = _mm_and_si128(_mm_srli_epi16(bytes, 4), nib);
      const __m512 q = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm_unpacklo_epi8(lo, hi)));
      _mm512_storeu_ps(wrow + i, cb_round_t16(_mm512_fmadd_ps(s, q, b), j->dtype));
    }
  }
}

__attribute__((target("avx512f,avx512bw,avx512vl"))) static float cb_dot_avx512(const float* a, const float* b,
                                                                               size_t k) {
  __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
  size_t i = 0;
  for (; i + 32 <= k; i += 32) {
    acc0 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), acc0);
    acc1 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i + 16), _mm512_loadu_ps(b + i + 16), acc1);
  }
  float t = _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
  for (; i < k; ++i) t += a[i] * b[i];
  return t;
}

static void* cb_worker(void* arg) {
  const cb_job* j = (const cb_job*)arg;
  const size_t k = j->k;
  float* xf = (float*)aligned_alloc(64, ((j->m * k * sizeof(float)) + 63) & ~(size_t)63);
  float* wrow = (float*)aligned_alloc(64, ((k * sizeof(float)) + 63) & ~(size_t)63);
  for (size_t i = 0; i < j->m * k; ++i) xf[i] = cb_to_f32(j->x[i], j->dtype);
  const int simd = j->bits == 4 && j->gs % 16 == 0 && j->form != CB_SCALAR;
  for (size_t r = j->n0; r < j->n1; ++r) {
    if (simd && j->form == CB_AVX512)
      cb_row_avx512(j, r, wrow);
    else if (simd && j->form == CB_AVX2)
      cb_row_avx2(j, r, wrow);
    else
      cb_row_scalar(j, r, wrow);
    for (size_t mi = 0; mi < j->m; ++mi) {
      const float* xr = xf + mi * k;
      float t;
      if (j->form == CB_AVX512)
        t = cb_dot_avx512(xr, wrow, k);
      else if (j->form == CB_AVX2)
        t = cb_dot_avx2(xr, wrow, k);
      else
        t = cb_dot_scalar(xr, wrow, k);
      j->y[mi * j->n + r] = cb_from_f32(t, j->dtype);
    }
  }
  free(xf);
  free(wrow);
  return NULL;
}

/* 1 when this host runs `form`. */
int cb_form_supported(int form) {
  __builtin_cpu_init();
  if (form == CB_SCALAR) return 1;
  if (form == CB_AVX2) return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  if (form == CB_AVX512)
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl");
  return 0;
}

/* y[m, n] = x[m, k] . dequant(w)^T in the given form; returns -1 when the
 * host lacks the form or the arguments are malformed. */
int cb_qmm(const uint16_t* x, size_t m, const uint32_t* w, const uint16_t* scales, const uint16_t* biases, size_t n,
           size_t k, int gs, int bits, int dtype, uint16_t* y, int threads, int form) {
  if (!cb_form_supported(form) || gs <= 0 || k % (size_t)gs != 0 || (bits != 2 && bits != 3 && bits != 4 &&
                                                                     bits != 5 && bits != 6 && bits != 8))
    return -1;
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  if ((size_t)threads > n) threads = n ? (int)n : 1;
  pthread_t tid[64];
  cb_job jobs[64];
  const size_t per = (n + (size_t)threads - 1) / (size_t)threads;
  for (int t = 0; t < threads; ++t) {
    const size_t n0 = (size_t)t * per < n ? (size_t)t * per : n;
    const size_t n1 = n0 + per < n ? n0 + per : n;
    jobs[t] = (cb_job){x, m, w, scales, biases, n0, n1, n, k, gs, bits, dtype, form, y};
    pthread_create(&tid[t], NULL, cb_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  return 0;
}
