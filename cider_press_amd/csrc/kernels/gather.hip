// Routed-expert quantized matmul, expert-major, for gfx950:
//   Y[r, :] = X[lhs[r], :] . dequant(W[rhs[r]])^T      (r < n_rows)
//
// Reference semantics: affine_gather_qmm_rhs / affine_gather_qmm_t
// (kernels-mlx/.../quantized.h:2092-2172, 2242-2436): each routed row is
// multiplied by its expert's weight, dequantized to T, fp32 accumulation.
//
// A workgroup (8 waves) owns one expert and one chunk of NC output columns.
// Per pass it gathers up to R = 16*MB of the rows routed to its expert (in row
// order: sorted routing by binary search, unsorted by per-64-row-block match
// counts, their prefix, and a ballot placement), stages those rows'
// activations in LDS once (16-byte chunks XOR-swizzled by row, conflict-free
// for the MFMA reads), and then streams the chunk's weights:
//   - wave w owns the 16-column slabs w, w+8, ... of the chunk; for each slab
//     it walks K in steps of 4 chunks (lane l: column l%16, chunk 4u + l/16),
//     4 steps of weights and their (scale, bias) in flight;
//   - each step is dequantized in registers (natural k order; the exact
//     single-FMA form when every lane's group allows it, else fmaf) into four
//     v_mfma_f32_16x16x32 B operands and multiplied against the MB 16-row
//     activation blocks read from LDS;
//   - at a slab's last step the 16 x R tile is stored.
// Weights stream from HBM exactly once per pass and activations are read
// from L2 once per workgroup, so the kernel runs at the weight stream's rate
// for routings with up to R rows per expert (more rows: more passes).
#include <algorithm>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int GX_WAVES = 8;
constexpr int GX_THREADS = 64 * GX_WAVES;
constexpr int GX_PF = 4;                   // steps in flight per wave (4 measured ~2 % faster than 8, 12 slower)
constexpr int GX_XBYTES = 128 * 1024;      // LDS for the staged activation rows
constexpr int GX_MAXBLK = 1024;            // 64-row routing blocks (n_rows <= 65536)

struct GxShared {
  int cnt[GX_MAXBLK];  // unsorted routing: matches of this expert per 64-row block, then prefix
  int rows[64];        // routed rows of the pass (-1: none)
  int xrow[64];        // their activation rows (-1: none / invalid)
  int total, lo;
};

template <int BITS>
struct GxStep {
  uint32_t w[BITS];
  uint32_t s, b;  // kept apart until used: combining them would wait for the loads
};

// Cursor over a wave's (slab, unit) steps: slab j of the wave is the 16-column
// slab wave + 8j of the chunk, unit u its chunks 4u .. 4u+3 (lane group g
// takes 4u + g).  Pointers advance incrementally (no per-step 64-bit math).
template <int BITS>
struct GxCursor {
  const uint32_t* wrow;
  const uint16_t* srow;
  const uint16_t* brow;
  int u, slab, col;
  __device__ __forceinline__ void next(int units, int my_slabs, size_t wstride, size_t gstride, int n) {
    if (++u == units) {
      u = 0;
      if (slab + 1 < my_slabs) {  // past the last slab: stay (clamped re-loads, never used)
        ++slab;
        col += 16 * GX_WAVES;
        const bool ok = col < n;
        wrow += ok ? wstride : 0;
        srow += ok ? gstride : 0;
        brow += ok ? gstride : 0;
      }
    }
  }
};

// Scale / bias words of QS consecutive steps (a "quad"), loaded at its first
// step when QS > 1: the QS * 128 / GSQ groups of the lane's column that the
// quad's 4 QS chunks span, in one 8- or 16-byte load each (QS = 1: one 2-byte
// load of each per step, in the step itself).  The quad's first unit is a
// multiple of QS, so the vector is aligned and inside the column's row.
struct GxSb {
  u32x4 s, b;
};

template <int QS, int GSQ>
struct GxQuad {
  static constexpr int kBytes = QS > 1 ? QS * 128 / GSQ * 2 : 0;
  static_assert(QS == 1 || kBytes == 8 || kBytes == 16, "quad vector of 8 or 16 bytes");
};

template <int BITS, int QS>
__device__ __forceinline__ void gx_load(const GxCursor<BITS>& c, GxStep<BITS>& dst, int chunks, int g,
                                        int gs_shift) {
  const int ch = min(4 * c.u + g, chunks - 1);
  load_chunk<BITS>(c.wrow, (size_t)ch, dst.w);
  if constexpr (QS == 1) {
    const int gi = (ch << 5) >> gs_shift;
    dst.s = c.srow[gi];
    dst.b = c.brow[gi];
  }
}

template <int BITS, int QS, int GSQ>
__device__ __forceinline__ void gx_load_sb(const GxCursor<BITS>& c, GxSb& v) {
  const int gi = (c.u * 128) / GSQ;  // first group of the quad
  if constexpr (GxQuad<QS, GSQ>::kBytes == 16) {
    v.s = *reinterpret_cast<const u32x4*>(c.srow + gi);
    v.b = *reinterpret_cast<const u32x4*>(c.brow + gi);
  } else {
    const u32x2 s2 = *reinterpret_cast<const u32x2*>(c.srow + gi);
    const u32x2 b2 = *reinterpret_cast<const u32x2*>(c.brow + gi);
    v.s = u32x4{s2[0], s2[1], 0u, 0u};
    v.b = u32x4{b2[0], b2[1], 0u, 0u};
  }
}

// The 16-bit scale or bias of quad step I for this lane (lane group g): group
// (128 I + 32 g) / GSQ of the quad.  GSQ = 64: word I, half g / 2 (per lane,
// `sel` picks it); GSQ = 128: word I / 2, half I % 2.
// (I is a constant once the step loop is unrolled.)
template <typename TT, int GSQ>
__device__ __forceinline__ float gx_sb_f32(const u32x4& v, int I, uint32_t sel) {
  if constexpr (GSQ == 64) {
    const uint32_t word = v[I];
    if constexpr (Sig16<TT>::bf16)
      return __uint_as_float(__builtin_amdgcn_perm(word, word, sel));
    else
      return TT::to_f32((uint16_t)__builtin_amdgcn_perm(word, word, sel));
  } else {
    const uint32_t word = v[I >> 1];
    return TT::to_f32((uint16_t)((I & 1) ? word >> 16 : word & 0xffffu));
  }
}

// Byte selector of gx_sb_f32 for lane group g (GSQ = 64): the 16-bit half
// g / 2 into the high half (bf16: the f32 bits) or the low half (f16).
template <typename TT>
__device__ __forceinline__ uint32_t gx_sb_sel(int g) {
  if constexpr (Sig16<TT>::bf16)
    return (g >> 1) ? 0x03020c0cu : 0x01000c0cu;
  else
    return (g >> 1) ? 0x0c0c0302u : 0x0c0c0100u;
}

// The first GX_PF steps of a wave's weight stream; `ld` ends past them.
template <int BITS, int QS, int GSQ>
__device__ __forceinline__ void gx_fill(GxCursor<BITS>& ld, GxStep<BITS> (&ring)[GX_PF],
                                        GxSb (&sbq)[GX_PF / QS], int units, int my_slabs, size_t wstride,
                                        size_t gstride, int n, int chunks, int g, int gs_shift) {
#pragma unroll
  for (int p = 0; p < GX_PF; ++p) {
    gx_load<BITS, QS>(ld, ring[p], chunks, g, gs_shift);
    if constexpr (QS > 1)
      if (p % QS == 0) gx_load_sb<BITS, QS, GSQ>(ld, sbq[p / QS]);
    ld.next(units, my_slabs, wstride, gstride, n);
  }
}

// First index i of the ascending a[0, n) with a[i] >= key (n if none), by one
// wave: each round splits the candidate range into 64 sub-ranges and counts
// the ones that end below key (a prefix, since a ascends) -- two rounds of
// loads for n <= 4096 instead of a serial bisection.
__device__ __forceinline__ int wave_lower_bound(const uint32_t* __restrict__ a, int n, uint32_t key, int lane) {
  int lo = 0, len = n;
  while (len > 1) {  // uniform
    const int step = (len + 63) / 64;
    const int last = lo + (lane + 1) * step - 1;  // last element of sub-range `lane`
    const bool below = last < lo + len && a[last] < key;
    const int c = __popcll(__ballot(below));
    lo += c * step;
    len = min(step, len - c * step);
  }
  if (len == 1 && a[lo] < key) ++lo;
  return lo;
}

template <typename TT, int BITS, int MB, bool FAST, int QS, int GSQ>
__device__ __forceinline__ void gx_stream(GxCursor<BITS> ld, GxCursor<BITS> cp, GxStep<BITS> (&ring)[GX_PF],
                                          GxSb (&sbq)[GX_PF / QS], int T, int units, int my_slabs, size_t wstride,
                                          size_t gstride, int n, int chunks, int gs_shift, int g, int nl,
                                          const unsigned char* xs, int k, const GxShared& sh, int mbl,
                                          uint16_t* __restrict__ y) {
  const int TP = (T + GX_PF - 1) / GX_PF * GX_PF;
  const uint32_t sel = gx_sb_sel<TT>(g);
  f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  GxSb curq;
  for (int t0 = 0; t0 < TP; t0 += GX_PF) {
#pragma unroll
    for (int p = 0; p < GX_PF; ++p) {
      const int t = t0 + p;
      const GxStep<BITS> cur = ring[p];
      if constexpr (QS > 1)
        if (p % QS == 0) curq = sbq[p / QS];
      gx_load<BITS, QS>(ld, ring[p], chunks, g, gs_shift);  // clamped past the end: no branch, no wait
      if constexpr (QS > 1)
        if (p % QS == 0) gx_load_sb<BITS, QS, GSQ>(ld, sbq[p / QS]);
      ld.next(units, my_slabs, wstride, gstride, n);
      const int c = 4 * cp.u + g;
      const bool live = t < T && c < chunks && cp.col < n;
      float sf = 0.f, bf = 0.f;
      if constexpr (QS == 1) {
        sf = TT::to_f32((uint16_t)cur.s);
        bf = TT::to_f32((uint16_t)cur.b);
      } else {
        sf = gx_sb_f32<TT, GSQ>(curq.s, p % QS, sel);
        bf = gx_sb_f32<TT, GSQ>(curq.b, p % QS, sel);
      }
      sf = live ? sf : 0.f;
      bf = live ? bf : 0.f;
      const float s16 = sf * 0.0625f;
      const float c0 = FAST ? fmaf(-1024.f, sf, bf) : 0.f, c1 = FAST ? fmaf(-64.f, sf, bf) : 0.f;
      u32x4 bop[4];
      bop[0] = dequant_slice<TT, BITS, FAST, 0>(cur.w, sf, s16, bf, c0, c1);
      bop[1] = dequant_slice<TT, BITS, FAST, 1>(cur.w, sf, s16, bf, c0, c1);
      bop[2] = dequant_slice<TT, BITS, FAST, 2>(cur.w, sf, s16, bf, c0, c1);
      bop[3] = dequant_slice<TT, BITS, FAST, 3>(cur.w, sf, s16, bf, c0, c1);
      const int cq = min(c, chunks - 1) * 4;  // first 16-byte chunk of this lane's 32 k
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        if (mb >= mbl) break;  // 16-row blocks past the pass's rows (wave-uniform)
        const unsigned char* xr = xs + (size_t)(16 * mb + nl) * k * 2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(xr + (size_t)(((cq + i) ^ nl) * 16));
          acc[mb] = Mfma16<TT>::run(a, bop[i], acc[mb]);
        }
      }
      if (cp.u == units - 1) {  // slab done (uniform)
        if (t < T && cp.col < n) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if (mb >= mbl) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int rl = 16 * mb + 4 * g + i;
              const int r = sh.rows[rl];
              if (r >= 0 && sh.xrow[rl] >= 0) y[(size_t)r * n + cp.col] = TT::from_f32(acc[mb][i]);
            }
          }
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      cp.next(units, my_slabs, wstride, gstride, n);
    }
  }
}

template <typename TT, int BITS, int MB, int QS, int GSQ>
__global__ __launch_bounds__(GX_THREADS) void gather_expert_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, int x_rows,
    const uint32_t* __restrict__ lhs, const uint32_t* __restrict__ rhs, int n_rows,
    uint16_t* __restrict__ y, int n, int k, int gs_shift, int sorted, int nc, int sb_vec,
    unsigned int* __restrict__ status) {
  constexpr int R = 16 * MB;
  __shared__ GxShared sh;
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];  // R x K activations
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const uint32_t e = blockIdx.y;
  const int c0 = blockIdx.x * nc;
  const int ncols = min(nc, n - c0);
  const int chunks = k >> 5;
  const int units = (chunks + 3) >> 2;
  const int G = k >> gs_shift;
  const size_t words_per_row = (size_t)k * BITS / 32;
  const uint32_t* we = w + (size_t)e * n * words_per_row;
  const uint16_t* se = scales + (size_t)e * n * G;
  const uint16_t* be = biases + (size_t)e * n * G;

  // 0. Index validation, spread over the grid: workgroup b checks rows
  //    b * GX_THREADS + tid (+ multiples of the grid's threads).  A row with
  //    an expert index past the experts or an activation index past X is
  //    zeroed here (no workgroup stores it: no expert matches the first, the
  //    second's expert skips it) and counted, as is every descent of a
  //    sorted routing.  The first row's indices are loaded now and checked
  //    when the workgroup is done, so the loads never wait.
  const int ck_stride = gridDim.x * gridDim.y * GX_THREADS;
  const int ck_r0 = (blockIdx.y * gridDim.x + blockIdx.x) * GX_THREADS + tid;
  uint32_t ck_re = 0u, ck_le = 0u, ck_next = 0xffffffffu;
  if (ck_r0 < n_rows) {
    ck_re = rhs[ck_r0];
    ck_le = lhs ? lhs[ck_r0] : 0u;
    if (sorted && ck_r0 + 1 < n_rows) ck_next = rhs[ck_r0 + 1];
  }
  auto check_rows = [&]() {
    for (int r = ck_r0; r < n_rows; r += ck_stride) {
      uint32_t re = ck_re, le = ck_le, nx = ck_next;
      if (r != ck_r0) {
        re = rhs[r];
        le = lhs ? lhs[r] : 0u;
        nx = sorted && r + 1 < n_rows ? rhs[r + 1] : 0xffffffffu;
      }
      const bool bad = re >= gridDim.y || (lhs && le >= (uint32_t)x_rows);
      if (bad)
        for (int j = 0; j < n; ++j) y[(size_t)r * n + j] = 0;
      if (bad || (sorted && re > nx)) atomicAdd(status, 1u);
    }
  };

  // 1. Rows routed to e.
  const int nblk = (n_rows + 63) >> 6;
  if (sorted) {
    // [lo, hi) = equal range of e in the ascending rhs; waves 0 and 1 search
    // its two ends at once.
    if (wave < 2) {
      const int b = wave_lower_bound(rhs, n_rows, e + (uint32_t)wave, lane);
      if (lane == 0) sh.cnt[wave] = b;
    }
    __syncthreads();
    if (tid == 0) {
      sh.lo = sh.cnt[0];
      sh.total = sh.cnt[1] - sh.cnt[0];
    }
  } else {
    for (int b = wave; b < nblk; b += GX_WAVES) {
      const int r = (b << 6) + lane;
      const unsigned long long mask = __ballot(r < n_rows && rhs[r] == e);
      if (lane == 0) sh.cnt[b] = __popcll(mask);
    }
    __syncthreads();
    if (tid == 0) {  // exclusive prefix over the blocks
      int run = 0;
      for (int b = 0; b < nblk; ++b) {
        const int c = sh.cnt[b];
        sh.cnt[b] = run;
        run += c;
      }
      sh.total = run;
      sh.lo = 0;
    }
  }
  __syncthreads();
  const int total = sh.total;
  if (total == 0) {  // uniform
    check_rows();
    return;
  }

  // Wave w's slabs: 16-column slabs w, w+8, ... of the chunk.  Their first
  // GX_PF weight steps are requested now, so the stream is in flight while
  // the constants are voted on and the activations staged.
  const int nslab = (ncols + 15) >> 4;
  const int my_slabs = nslab > wave ? (nslab - wave + GX_WAVES - 1) / GX_WAVES : 0;
  const int T = my_slabs * units;  // live steps of this wave
  const size_t wstride = (size_t)16 * GX_WAVES * words_per_row, gstride = (size_t)16 * GX_WAVES * G;
  GxCursor<BITS> start;
  start.u = 0;
  start.slab = 0;
  start.col = c0 + 16 * wave + nl;
  const int col0 = min(start.col, n - 1);
  start.wrow = we + (size_t)col0 * words_per_row;
  start.srow = se + (size_t)col0 * G;
  start.brow = be + (size_t)col0 * G;
  GxStep<BITS> ring[GX_PF];
  GxSb sbq[GX_PF / QS];
  GxCursor<BITS> ld = start;
  if (T > 0) gx_fill<BITS, QS, GSQ>(ld, ring, sbq, units, my_slabs, wstride, gstride, n, chunks, g, gs_shift);

  // 2. Fast-path vote over the chunk's (column, group) pairs.  The chunk's
  //    columns are consecutive rows of the expert's [n, G] tables, so its
  //    pairs are one contiguous run of ncols * G entries: 16-byte segments
  //    (when the run starts 16-byte aligned) get the packed exponent check,
  //    and the exact predicate where that one does not clear a thread's
  //    segments; the tail and unaligned runs go pair by pair.
  bool ok = true;
  const size_t run0 = (size_t)c0 * G;
  const int run = ncols * G;
  const int nvec = sb_vec ? run >> 3 : 0;
  for (int i0 = tid; i0 < nvec; i0 += 4 * GX_THREADS) {
    u32x4 sv[4], bv[4];
    bool live[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int i = i0 + h * GX_THREADS;
      live[h] = i < nvec;
      if (live[h]) {
        sv[h] = *reinterpret_cast<const u32x4*>(se + run0 + (size_t)i * 8);
        bv[h] = *reinterpret_cast<const u32x4*>(be + run0 + (size_t)i * 8);
      } else {  // a pair the packed check accepts
        sv[h] = bv[h] = u32x4{0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};
      }
    }
    FastQuick fq;
    fast_quick_init(fq);
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) fast_quick_add<TT>(fq, sv[h][q], bv[h][q]);
    if (!fast_quick_ok<TT>(fq)) {
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ok &= !live[h] | (fast_ok_bits<TT>(sv[h][q] & 0xffffu, bv[h][q] & 0xffffu) &
                            fast_ok_bits<TT>(sv[h][q] >> 16, bv[h][q] >> 16));
    }
  }
  for (int i = 8 * nvec + tid; i < run; i += GX_THREADS) ok &= fast_ok_bits<TT>(se[run0 + i], be[run0 + i]);
  bool fast = __syncthreads_and(ok);
  if constexpr (BITS != 4 && BITS != 8) fast = false;

  for (int p0 = 0; p0 < total; p0 += R) {
    // 3. The pass's rows and activation rows.
    if (tid < R) sh.rows[tid] = -1;
    __syncthreads();
    if (sorted) {
      if (tid < R && p0 + tid < total) sh.rows[tid] = sh.lo + p0 + tid;
    } else {
      for (int b = wave; b < nblk; b += GX_WAVES) {
        const int base = sh.cnt[b];
        const int next = b + 1 < nblk ? sh.cnt[b + 1] : total;
        if (next <= p0 || base >= p0 + R) continue;  // uniform per wave
        const int r = (b << 6) + lane;
        const bool match = r < n_rows && rhs[r] == e;
        const unsigned long long mask = __ballot(match);
        const int rank = base + __popcll(mask & ((1ull << lane) - 1ull));
        if (match && rank >= p0 && rank < p0 + R) sh.rows[rank - p0] = r;
      }
    }
    __syncthreads();
    if (tid < R) {
      const int r = sh.rows[tid];
      int xi = -1;
      if (r >= 0) {
        const uint32_t v = lhs ? lhs[r] : (uint32_t)r;
        if (v < (uint32_t)x_rows) xi = (int)v;
      }
      sh.xrow[tid] = xi;
    }
    __syncthreads();

    // 4. Activation rows into LDS in the dequantizer's slot order, 16-byte
    //    chunk q of row i at i*K*2 + (q ^ (i & 15))*16.  Only the pass's
    //    rows are staged, 8 loads per thread in flight: the other rows of
    //    its 16-row blocks keep stale LDS bytes, which reach only their own
    //    output rows (MFMA rows are independent), and those are not stored.
    const int kq = k >> 3;  // 16-byte chunks per row
    const int nst = min(R, total - p0) * kq;
    for (int idx = tid; idx < nst; idx += GX_THREADS * 8) {
      u32x4 v[8];
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        const int id = idx + h * GX_THREADS;
        v[h] = u32x4{0u, 0u, 0u, 0u};
        if (id < nst) {
          const int i = id / kq, q = id - i * kq;
          const int xi = sh.xrow[i];
          if (xi >= 0) v[h] = *reinterpret_cast<const u32x4*>(x + (size_t)xi * k + (size_t)q * 8);
        }
      }
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        const int id = idx + h * GX_THREADS;
        if (id < nst) {
          const int i = id / kq, q = id - i * kq;
          *reinterpret_cast<u32x4*>(xs + (size_t)i * k * 2 + (size_t)((q ^ (i & 15)) * 16)) =
              interleave_x<BITS>(v[h]);
        }
      }
    }
    __syncthreads();

    // 5. Stream the weights of this wave's slabs; only the 16-row blocks
    //    that hold rows of this pass are multiplied.
    const int mbl = (min(R, total - p0) + 15) >> 4;
    if (T > 0) {
      if (p0 > 0) {  // a further pass streams the weights again
        ld = start;
        gx_fill<BITS, QS, GSQ>(ld, ring, sbq, units, my_slabs, wstride, gstride, n, chunks, g, gs_shift);
      }
      if (fast)
        gx_stream<TT, BITS, MB, true, QS, GSQ>(ld, start, ring, sbq, T, units, my_slabs, wstride, gstride, n, chunks, gs_shift,
                                      g, nl, xs, k, sh, mbl, y);
      else
        gx_stream<TT, BITS, MB, false, QS, GSQ>(ld, start, ring, sbq, T, units, my_slabs, wstride, gstride, n, chunks,
                                       gs_shift, g, nl, xs, k, sh, mbl, y);
    }
    __syncthreads();  // LDS rows / activations are rewritten by the next pass
  }
  check_rows();
}

template <typename TT, int BITS, int MB, int QS, int GSQ>
hipError_t launch_q(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                    const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                    int gs_shift, int n_chunks, int nc, int sb_vec, unsigned int* status) {
  static const hipError_t attr = [] {
    const void* fn = reinterpret_cast<const void*>(&gather_expert_kernel<TT, BITS, MB, QS, GSQ>);
    hipFuncAttributes fa;
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(160 * 1024 - fa.sharedSizeBytes));
  }();
  if (attr != hipSuccess) return attr;
  const size_t lds = (size_t)16 * MB * k * 2;
  hipLaunchKernelGGL((gather_expert_kernel<TT, BITS, MB, QS, GSQ>), dim3((unsigned)n_chunks, (unsigned)n_experts),
                     dim3(GX_THREADS), lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x), x_rows, lhs,
                     rhs, n_rows, static_cast<uint16_t*>(y), n, k, gs_shift, (int)sorted, nc, sb_vec, status);
  return hipGetLastError();
}

// Scale / bias quads: 4 steps per 16-byte load (gs 64) or 8-byte load (gs
// 128) when a slab's units divide by 4, else 2 steps per 8-byte load (gs 64),
// else per-step 2-byte loads.  Alignment: row starts are multiples of the
// vector (G a multiple of its groups) and the base pointers aligned to it.
template <typename TT, int BITS, int MB>
hipError_t launch_mb(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                     const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                     int gs_shift, int n_chunks, int nc, unsigned int* status) {
  const int G = k / q.gs, units = k / 128;
  const uintptr_t al = reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases);
  // Vote runs start at (e n + c0) G entries, c0 a multiple of 128.
  const int sb_vec = ((long)n * G % 8 == 0) && (al % 16 == 0);
  static const int forced = env_int("CPQ_GATHER_QS", 0);
#define CPQ_GXQ(QS, GSQ)                                                                                  \
  return launch_q<TT, BITS, MB, QS, GSQ>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted,   \
                                         gs_shift, n_chunks, nc, sb_vec, status)
  if (forced != 1) {
    if (q.gs == 64 && units % 4 == 0 && al % 16 == 0 && forced != 2) CPQ_GXQ(4, 64);
    if (q.gs == 64 && units % 2 == 0 && al % 8 == 0) CPQ_GXQ(2, 64);
    if (q.gs == 128 && units % 4 == 0 && al % 8 == 0) CPQ_GXQ(4, 128);
  }
  CPQ_GXQ(1, 64);
#undef CPQ_GXQ
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                    const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                    int cu_count, unsigned int* status) {
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  // Column chunks (whole multiples of 8 slabs = 128 columns): the count that
  // minimises rounds-of-workgroups x work-per-workgroup over the CUs.
  const int slabs128 = (n + 127) / 128;
  int best = 1;
  long best_cost = -1;
  for (int c = 1; c <= slabs128; ++c) {
    const long rounds = ((long)c * n_experts + cu_count - 1) / cu_count;
    const long cost = rounds * ((slabs128 + c - 1) / c);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = c;
    }
  }
  const int nc = (slabs128 + best - 1) / best * 128;
  const int n_chunks = (n + nc - 1) / nc;
  if ((size_t)64 * k * 2 <= (size_t)GX_XBYTES)
    return launch_mb<TT, BITS, 4>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, gs_shift,
                                  n_chunks, nc, status);
  if ((size_t)32 * k * 2 <= (size_t)GX_XBYTES)
    return launch_mb<TT, BITS, 2>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, gs_shift,
                                  n_chunks, nc, status);
  return launch_mb<TT, BITS, 1>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, gs_shift,
                                n_chunks, nc, status);
}

}  // namespace

bool gather_expert_supported(int bits, int n_rows, int k) {
  // k % 128: whole 16-chunk swizzle groups per staged row.
  return (bits == 4 || bits == 8) && k % 128 == 0 && n_rows <= 64 * GX_MAXBLK &&
         (size_t)16 * k * 2 <= (size_t)GX_XBYTES;
}

hipError_t launch_gather_expert(hipStream_t s, const QuantArgs& q, const void* x, int x_rows,
                                const uint32_t* lhs, const uint32_t* rhs, int n_rows, void* y,
                                int n_experts, int n, int k, bool sorted, int cu_count,
                                unsigned int* status) {
#define CPQ_GX(TT)                                                                                        \
  switch (q.bits) {                                                                                       \
    case 4: return launch_t<TT, 4>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, cu_count, status); \
    case 8: return launch_t<TT, 8>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, cu_count, status); \
    default: return hipErrorInvalidValue;                                                                 \
  }
  if (q.dtype == CPQ_DTYPE_BF16) { CPQ_GX(BF16) }
  if (q.dtype == CPQ_DTYPE_F16) { CPQ_GX(F16) }
#undef CPQ_GX
  return hipErrorInvalidValue;
}

}  // namespace cpq
