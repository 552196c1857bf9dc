/*
 * cpq_oracle.c -- CPU restatement of the reference's affine group-quantized
 * matmul path (MLX-style packing, per-group scale and bias, w = scale*q + bias).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The HIP library (cider_press_amd/libcpq.so) never links it.
 *
 * Reference files followed (paths relative to the reference checkout):
 *   kernels-mlx/mlx/backend/metal/kernels/quantized.h
 *     :17-26      pack factor / bytes per pack
 *     :28-104     load_vector (x pre-division, T-typed 4-sums)
 *     :191-290    qdot (masked, unshifted nibbles; scale*accum + sum*bias)
 *     :749-814    qmv_fast_impl (16 values/thread for 4-bit, 512 block)
 *     :816-975    qmv_impl (generic tiling with safe tail)
 *     :1087-1213  qmm_t_impl (dequantize tile to T, fp32 accumulate)
 *     :2092-2172, 2242-2436  gather_qmm_t / gather_qmm_rhs (per-row expert)
 *     :2543-2603  affine_dequantize (LE bit stream, out = scale*q + bias)
 *   crates/cider-press-kernels/src/kernels/qmv.rs:165-172 (fast/generic rule)
 *
 * Pinning (see tests/test_oracle.py):
 *   or_qmv_mlx          -- bit-exact against the reference's committed golden
 *                          crates/cider-press-kernels/tests/fixtures/qmv.safetensors
 *                          and near-exact on qmm_qwen2.safetensors.
 *   or_unpack_row       -- the same goldens (a wrong nibble order fails them),
 *                          plus an independent numpy bit-stream unpack.
 *   or_dequantize       -- special cases q=0 -> RNE(b), b=-8s -> RNE(s(q-8)),
 *                          and torch's RNE bf16/f16 conversions of numpy fp32 fma.
 *   or_qmm_ref          -- numpy float64 matmul of independently dequantized W,
 *                          brute force on tiny shapes, linearity.
 *   or_gather_qmm_ref   -- reduction to or_qmm_ref row by row.
 *   f32<->bf16/f16      -- torch / numpy RNE conversions on exhaustive patterns.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2 };

/* ------------------------------------------------------------------ */
/* Scalar conversions (IEEE round-to-nearest-even).                    */
/* ------------------------------------------------------------------ */

float or_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  float f;
  if (e == 0) {
    /* zero or subnormal: m * 2^-24, exact in f32 */
    f = (float)m * 5.9604644775390625e-08f;
    if (sign) f = -f;
    return f;
  }
  uint32_t u;
  if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e - 15u + 127u) << 23) | (m << 13);
  }
  memcpy(&f, &u, 4);
  return f;
}

uint16_t or_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t a = x & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);     /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);    /* >= 65520 -> inf */
  if (a < 0x38800000u) {                                       /* below 2^-14 */
    float v;
    memcpy(&v, &a, 4);
    float t = v * 16777216.0f; /* v / 2^-24, exact */
    uint32_t m = (uint32_t)rintf(t); /* default rounding mode: nearest-even */
    return (uint16_t)(sign | m);
  }
  uint32_t e = (a >> 23) - 127u + 15u;
  uint32_t mant = a & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

static inline float to_f32(uint16_t v, int dtype) {
  return dtype == OR_BF16 ? or_bf16_to_f32(v) : or_f16_to_f32(v);
}
static inline uint16_t from_f32(float v, int dtype) {
  return dtype == OR_BF16 ? or_f32_to_bf16(v) : or_f32_to_f16(v);
}
/* Round an f32 to T and back: the value a T-typed register holds. */
static inline float round_t(float v, int dtype) { return to_f32(from_f32(v, dtype), dtype); }

/* ------------------------------------------------------------------ */
/* Packing: element i of a row occupies bits [bits*i, bits*(i+1)) of   */
/* the row's little-endian bit stream (quantized.h:2565-2600; for      */
/* bits in {2,4,8} this is (word >> bits*j) & mask, :2589-2600).       */
/* ------------------------------------------------------------------ */

void or_unpack_row(const uint32_t* row, int bits, size_t k, uint8_t* q) {
  const uint32_t mask = (1u << bits) - 1u;
  for (size_t i = 0; i < k; ++i) {
    size_t bit = i * (size_t)bits;
    size_t wi = bit >> 5;
    unsigned off = (unsigned)(bit & 31u);
    uint32_t v = row[wi] >> off;
    if (off + (unsigned)bits > 32u) v |= row[wi + 1] << (32u - off);
    q[i] = (uint8_t)(v & mask);
  }
}

/* Pack values (each < 2^bits) into a zeroed row of K*bits/32 words. */
void or_pack_row(const uint8_t* q, int bits, size_t k, uint32_t* row) {
  size_t words = k * (size_t)bits / 32u;
  memset(row, 0, words * 4u);
  for (size_t i = 0; i < k; ++i) {
    size_t bit = i * (size_t)bits;
    size_t wi = bit >> 5;
    unsigned off = (unsigned)(bit & 31u);
    row[wi] |= (uint32_t)q[i] << off;
    if (off + (unsigned)bits > 32u) row[wi + 1] |= (uint32_t)q[i] >> (32u - off);
  }
}

/* ------------------------------------------------------------------ */
/* Dequantize (quantized.h:2543-2603).  Contract: out = RNE_T(fmaf(s,q,b)),  */
/* one f32 rounding then one rounding to T.                              */
/* ------------------------------------------------------------------ */

void or_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                   size_t rows, size_t k, int gs, int bits, int dtype, uint16_t* out) {
  size_t words_per_row = k * (size_t)bits / 32u;
  size_t groups_per_row = k / (size_t)gs;
  uint8_t* q = (uint8_t*)malloc(k);
  for (size_t r = 0; r < rows; ++r) {
    or_unpack_row(w + r * words_per_row, bits, k, q);
    for (size_t i = 0; i < k; ++i) {
      size_t g = r * groups_per_row + i / (size_t)gs;
      float s = to_f32(scales[g], dtype);
      float b = to_f32(biases[g], dtype);
      out[r * k + i] = from_f32(fmaf(s, (float)q[i], b), dtype);
    }
  }
  free(q);
}

/* Dequantize rows to f32 (the values of the T-rounded weights). */
static void dequant_rows_f32(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                             size_t r0, size_t r1, size_t k, int gs, int bits, int dtype,
                             float* out /* (r1-r0) x k */) {
  size_t words_per_row = k * (size_t)bits / 32u;
  size_t groups_per_row = k / (size_t)gs;
  uint8_t* q = (uint8_t*)malloc(k);
  for (size_t r = r0; r < r1; ++r) {
    or_unpack_row(w + r * words_per_row, bits, k, q);
    float* o = out + (r - r0) * k;
    for (size_t i = 0; i < k; ++i) {
      size_t g = r * groups_per_row + i / (size_t)gs;
      float s = to_f32(scales[g], dtype);
      float b = to_f32(biases[g], dtype);
      o[i] = round_t(fmaf(s, (float)q[i], b), dtype);
    }
  }
  free(q);
}

/* ------------------------------------------------------------------ */
/* Reference matmul: Y[m,n] = sum_k X[m,k] * dequant(W)[n,k]             */
/* (quantized.h:1087-1213: dequantize to T, accumulate wide).  Output    */
/* is unrounded float64.  Multithreaded over N.                          */
/* ------------------------------------------------------------------ */

typedef struct {
  const uint16_t* x; size_t m;
  const uint32_t* w; const uint16_t* s; const uint16_t* b;
  size_t n0, n1, n, k; int gs, bits, dtype;
  double* y;
} qmm_job;

static void* qmm_ref_worker(void* arg) {
  qmm_job* j = (qmm_job*)arg;
  const size_t CH = 16;
  float* wd = (float*)malloc(CH * j->k * sizeof(float));
  double* xd = (double*)malloc(j->m * j->k * sizeof(double));
  for (size_t i = 0; i < j->m * j->k; ++i) xd[i] = (double)to_f32(j->x[i], j->dtype);
  for (size_t r0 = j->n0; r0 < j->n1; r0 += CH) {
    size_t r1 = r0 + CH < j->n1 ? r0 + CH : j->n1;
    dequant_rows_f32(j->w, j->s, j->b, r0, r1, j->k, j->gs, j->bits, j->dtype, wd);
    for (size_t mi = 0; mi < j->m; ++mi) {
      const double* xr = xd + mi * j->k;
      for (size_t r = r0; r < r1; ++r) {
        const float* wr = wd + (r - r0) * j->k;
        /* Four float64 partial sums (k mod 4) combined at the end: the
         * products are exact in float64, and four independent chains keep
         * the full-size references of the benchmark shapes affordable. */
        double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
        size_t kk = 0;
        for (; kk + 4 <= j->k; kk += 4) {
          a0 += xr[kk] * (double)wr[kk];
          a1 += xr[kk + 1] * (double)wr[kk + 1];
          a2 += xr[kk + 2] * (double)wr[kk + 2];
          a3 += xr[kk + 3] * (double)wr[kk + 3];
        }
        for (; kk < j->k; ++kk) a0 += xr[kk] * (double)wr[kk];
        j->y[mi * j->n + r] = (a0 + a1) + (a2 + a3);
      }
    }
  }
  free(wd);
  free(xd);
  return NULL;
}

static int clamp_threads(int t, size_t work) {
  if (t < 1) t = 1;
  if (t > 64) t = 64;
  if ((size_t)t > work) t = (int)(work ? work : 1);
  return t;
}

void or_qmm_ref(const uint16_t* x, size_t m, const uint32_t* w, const uint16_t* scales,
                const uint16_t* biases, size_t n, size_t k, int gs, int bits, int dtype,
                double* y, int threads) {
  threads = clamp_threads(threads, n);
  pthread_t tid[64];
  qmm_job jobs[64];
  size_t per = (n + (size_t)threads - 1) / (size_t)threads;
  for (int t = 0; t < threads; ++t) {
    size_t n0 = (size_t)t * per, n1 = n0 + per < n ? n0 + per : n;
    jobs[t] = (qmm_job){x, m, w, scales, biases, n0 < n ? n0 : n, n1, n, k, gs, bits, dtype, y};
    pthread_create(&tid[t], NULL, qmm_ref_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------------ */
/* Gather: Y[r,n] = sum_k X[lhs[r],k] * dequant(W[rhs[r]])[n,k]          */
/* (quantized.h:1390-1442 picks x row and expert per batch item;          */
/* :2242-2436 walks runs of equal expert index).  lhs may be NULL         */
/* (identity).  Expert e occupies rows [e*n, (e+1)*n) of w/scales/biases. */
/* ------------------------------------------------------------------ */

void or_gather_qmm_ref(const uint16_t* x, const uint32_t* lhs, const uint32_t* rhs,
                       size_t rows, const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, size_t n, size_t k, int gs, int bits,
                       int dtype, double* y, int threads) {
  size_t words_per_expert = n * k * (size_t)bits / 32u;
  size_t groups_per_expert = n * (k / (size_t)gs);
  /* Rows are grouped by expert so each expert is dequantized once: the rows
   * of expert e are gathered into one activation block and reduced by
   * or_qmm_ref (the per-element sums are the same as row by row). */
  size_t* order = (size_t*)malloc((rows ? rows : 1) * sizeof(size_t));
  uint16_t* xb = (uint16_t*)malloc((rows ? rows : 1) * k * sizeof(uint16_t));
  double* yb = (double*)malloc((rows ? rows : 1) * n * sizeof(double));
  uint8_t* done = (uint8_t*)calloc(rows ? rows : 1, 1);
  for (size_t r0 = 0; r0 < rows; ++r0) {
    if (done[r0]) continue;
    const size_t e = rhs[r0];
    size_t cnt = 0;
    for (size_t r = r0; r < rows; ++r)
      if (!done[r] && rhs[r] == e) {
        order[cnt] = r;
        done[r] = 1;
        const size_t xr = lhs ? lhs[r] : r;
        memcpy(xb + cnt * k, x + xr * k, k * sizeof(uint16_t));
        ++cnt;
      }
    or_qmm_ref(xb, cnt, w + e * words_per_expert, scales + e * groups_per_expert,
               biases + e * groups_per_expert, n, k, gs, bits, dtype, yb, threads);
    for (size_t i = 0; i < cnt; ++i) memcpy(y + order[i] * n, yb + i * n, n * sizeof(double));
  }
  free(order);
  free(xb);
  free(yb);
  free(done);
}

/* ------------------------------------------------------------------ */
/* MLX qmv arithmetic, restated (quantized.h:28-104, 191-290, 749-975).   */
/* Each of 32 simd lanes owns `vpt` consecutive values of every block of  */
/* 32*vpt; it keeps x pre-divided by 16^j (4-bit) / 4^j (2-bit), sums x   */
/* in chunks of four added in T arithmetic (:40,64), and returns          */
/* scale*accum + sum*bias per block (:289).  Lane partials are combined   */
/* by a butterfly (simd_sum) and rounded to T.  Output y_f32 is the       */
/* unrounded f32 value before the final cast.                             */
/* Supports bits in {2, 4, 8}; `fast` selects qmv_fast (2 packs/thread,   */
/* 1 for 2-bit) vs qmv (1 pack/thread), per qmv.rs:165-172.              */
/* ------------------------------------------------------------------ */

int or_qmv_mlx(const uint16_t* x, size_t m, const uint32_t* w, const uint16_t* scales,
               const uint16_t* biases, size_t n, size_t k, int gs, int bits, int dtype,
               int fast, float* y_f32) {
  if (bits != 2 && bits != 4 && bits != 8) return -1;
  const int pack_factor = 32 / bits;                       /* values per u32 */
  const int packs_per_thread = fast ? (bits == 2 ? 1 : 2) : 1;
  const int vpt = pack_factor * packs_per_thread;          /* values per thread */
  const int block = vpt * 32;
  size_t words_per_row = k * (size_t)bits / 32u;
  size_t groups_per_row = k / (size_t)gs;
  uint8_t* q = (uint8_t*)malloc(k);
  float xt[64];
  for (size_t mi = 0; mi < m; ++mi) {
    const uint16_t* xr = x + mi * k;
    for (size_t r = 0; r < n; ++r) {
      or_unpack_row(w + r * words_per_row, bits, k, q);
      float lane[32];
      for (int t = 0; t < 32; ++t) {
        float result = 0.0f;
        for (size_t kb = 0; kb < k; kb += (size_t)block) {
          size_t base = kb + (size_t)t * (size_t)vpt;
          if (base >= k) continue;
          int cnt = (int)((k - base) < (size_t)vpt ? (k - base) : (size_t)vpt);
          /* load_vector / load_vector_safe */
          float sum = 0.0f;
          if (bits == 8) {
            for (int i = 0; i < cnt; ++i) {
              float xv = to_f32(xr[base + i], dtype);
              sum += xv;
              xt[i] = xv;
            }
          } else {
            const float d1 = bits == 4 ? 16.0f : 4.0f;
            const float d2 = bits == 4 ? 256.0f : 16.0f;
            const float d3 = bits == 4 ? 4096.0f : 64.0f;
            for (int i = 0; i < cnt; i += 4) {
              float x0 = to_f32(xr[base + i], dtype), x1 = to_f32(xr[base + i + 1], dtype);
              float x2 = to_f32(xr[base + i + 2], dtype), x3 = to_f32(xr[base + i + 3], dtype);
              float c = round_t(x0 + x1, dtype); /* T + T -> T */
              c = round_t(c + x2, dtype);
              c = round_t(c + x3, dtype);
              sum += c;
              xt[i] = x0;
              xt[i + 1] = x1 / d1;
              xt[i + 2] = x2 / d2;
              xt[i + 3] = x3 / d3;
            }
          }
          /* qdot / qdot_safe: masked but unshifted sub-fields */
          float accum = 0.0f;
          if (bits == 8) {
            for (int i = 0; i < cnt; ++i) accum += xt[i] * (float)q[base + i];
          } else {
            const int sh = bits; /* positions within each 4-value chunk */
            for (int i = 0; i < cnt; i += 4) {
              float p0 = xt[i] * (float)((uint32_t)q[base + i]);
              float p1 = xt[i + 1] * (float)((uint32_t)q[base + i + 1] << sh);
              float p2 = xt[i + 2] * (float)((uint32_t)q[base + i + 2] << (2 * sh));
              float p3 = xt[i + 3] * (float)((uint32_t)q[base + i + 3] << (3 * sh));
              accum += ((p0 + p1) + p2) + p3;
            }
          }
          size_t g = r * groups_per_row + base / (size_t)gs;
          float s = to_f32(scales[g], dtype);
          float b = to_f32(biases[g], dtype);
          result += s * accum + sum * b;
        }
        lane[t] = result;
      }
      for (int off = 16; off >= 1; off >>= 1) {
        float nv[32];
        for (int t = 0; t < 32; ++t) nv[t] = lane[t] + lane[t ^ off];
        memcpy(lane, nv, sizeof(nv));
      }
      y_f32[mi * n + r] = lane[0];
    }
  }
  free(q);
  return 0;
}
