// Small-M quantized GEMM and routed-expert gather for gfx950.
//
//   skinny:  Y[M,N] = X[M,K] . dequant(W[N,K])^T for M up to a few dozen rows.
//   gather:  Y[r,:] = X[lhs[r],:] . dequant(W[rhs[r]])^T   (routed experts).
//
// Reference semantics: qmm_t_impl (kernels-mlx/.../quantized.h:1087-1213) for
// the dense case and affine_gather_qmm_rhs / affine_gather_qmm_t
// (quantized.h:2092-2172, 2242-2436) for the gather case: dequantize W to T,
// accumulate in fp32, store T.
//
// Both are HBM-bound (the weight stream dominates), so a weight is read and
// dequantized exactly once per workgroup and then multiplied against every
// activation row on the matrix cores:
//   - workgroup = 4 waves, one 16-column slab of W (16 output columns);
//   - each wave walks a quarter of K in 128-element steps; lane l loads the
//     32-element chunk (bits words, 16 B at 4-bit) of row n0 + l%16 at chunk
//     4u + l/16, dequantizes it in registers into four 8-element MFMA
//     B-operand slices, and issues v_mfma_f32_16x16x32_{bf16,f16} against
//     up to MB 16-row blocks of activations (A operand read straight from
//     global/L2: activations are tiny next to W);
//   - the four K-partial 16x16 tiles are summed through LDS.
// MFMA 16x16x32 operand layout: A[m][k] in lane m + 16*(k/8), element k%8;
// B[k][n] in lane n + 16*(k/8), element k%8; D[m][n] in lane n + 16*(m/4),
// element m%4.  Any bijection of k onto (lane group, element) is valid as long
// as A and B agree; lane group g / slice i / element j <-> k = 32*(4u+g)+8i+j.
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int kMaxMB = 4;  // up to 64 activation rows per pass

// WAVES waves split K; MBS row blocks of 16 activation rows per pass.
template <int WAVES, int MBS>
struct TileShared {
  const uint16_t* xrow[16 * MBS];  // activation row per local row (nullptr: zero row)
  uint16_t* yrow[16 * MBS];        // output row per local row (nullptr: not stored)
  float red[WAVES][MBS][64][4];    // K-partial tiles
  int rows[16 * kMaxMB];              // gather: global row ids of this pass
  int count;
  int pos;
};

// Per-(column, group) constants (s, b, b - 1024 s, b - 64 s) of a 16-column
// slab, gc[col * GP + g], and the workgroup's fast-path vote.  Split in two so
// the caller can put the weight prefetch between the loads and their use:
// slab_consts_load issues the loads (16-byte vectors of 8 groups when the
// layout allows), slab_consts_store writes LDS, votes and ends in a barrier.
constexpr int kConstSlots = 2;  // 16-byte segments per thread held in registers

struct SlabConsts {
  u32x4 sv[kConstSlots], bv[kConstSlots];
};

template <int NT>
__device__ __forceinline__ void slab_consts_load(const uint16_t* __restrict__ scales,
                                                 const uint16_t* __restrict__ biases, int n, int G,
                                                 int n0, bool vec, SlabConsts& sc) {
  const int segs = G >> 3;
#pragma unroll
  for (int t = 0; t < kConstSlots; ++t) {
    sc.sv[t] = sc.bv[t] = u32x4{0u, 0u, 0u, 0u};
    const int i = threadIdx.x + NT * t;
    if (vec && i < 16 * segs) {
      const int c = i / segs, sg = i - c * segs;
      if (n0 + c < n) {
        sc.sv[t] = *reinterpret_cast<const u32x4*>(scales + (size_t)(n0 + c) * G + sg * 8);
        sc.bv[t] = *reinterpret_cast<const u32x4*>(biases + (size_t)(n0 + c) * G + sg * 8);
      }
    }
  }
}

template <typename TT, int NT>
__device__ __forceinline__ bool slab_consts_store(const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases, int n, int G,
                                                  int n0, bool vec, const SlabConsts& sc, f32x4* gc,
                                                  int GP) {
  bool ok = true;
  auto put = [&](int c, int gi, uint32_t sv, uint32_t bv) {
    const float sf = TT::to_f32((uint16_t)sv), bf = TT::to_f32((uint16_t)bv);
    gc[c * GP + gi] = f32x4{sf, bf, fmaf(-1024.f, sf, bf), fmaf(-64.f, sf, bf)};
  };
  // A 16-byte segment (8 groups): the packed exponent check, and the exact
  // predicate per group only when that one does not clear the segment.
  auto put8 = [&](int c, int sg, const u32x4& s4, const u32x4& b4) {
    FastQuick fq;
    fast_quick_init(fq);
#pragma unroll
    for (int q = 0; q < 4; ++q) fast_quick_add<TT>(fq, s4[q], b4[q]);
    if (!fast_quick_ok<TT>(fq)) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ok &= fast_ok_bits<TT>(s4[q] & 0xffffu, b4[q] & 0xffffu) & fast_ok_bits<TT>(s4[q] >> 16, b4[q] >> 16);
    }
#pragma unroll
    for (int h = 0; h < 8; ++h)
      put(c, sg * 8 + h, (h & 1) ? s4[h >> 1] >> 16 : s4[h >> 1] & 0xffffu,
          (h & 1) ? b4[h >> 1] >> 16 : b4[h >> 1] & 0xffffu);
  };
  if (vec) {
    const int segs = G >> 3;
#pragma unroll
    for (int t = 0; t < kConstSlots; ++t) {
      const int i = threadIdx.x + NT * t;
      if (i < 16 * segs) {
        const int c = i / segs, sg = i - c * segs;
        put8(c, sg, sc.sv[t], sc.bv[t]);
      }
    }
    for (int i = threadIdx.x + NT * kConstSlots; i < 16 * segs; i += NT) {
      const int c = i / segs, sg = i - c * segs;
      u32x4 s4 = {0u, 0u, 0u, 0u}, b4 = {0u, 0u, 0u, 0u};
      if (n0 + c < n) {
        s4 = *reinterpret_cast<const u32x4*>(scales + (size_t)(n0 + c) * G + sg * 8);
        b4 = *reinterpret_cast<const u32x4*>(biases + (size_t)(n0 + c) * G + sg * 8);
      }
      put8(c, sg, s4, b4);
    }
  } else {
    for (int it = threadIdx.x; it < 16 * G; it += NT) {
      const int c = it / G, gi = it - c * G;
      uint32_t sv = 0u, bv = 0u;
      if (n0 + c < n) {
        sv = scales[(size_t)(n0 + c) * G + gi];
        bv = biases[(size_t)(n0 + c) * G + gi];
      }
      ok &= fast_ok_bits<TT>(sv, bv);
      put(c, gi, sv, bv);
    }
  }
  return __syncthreads_and(ok);
}

// One 16-column slab of W against up to 16*MB activation rows (pointers in
// sh).  Each wave streams a contiguous quarter of K: PF weight chunks and the
// next step's activation slices stay in flight while a step is dequantized
// (natural k order) and multiplied.  Steps past the wave's range read clamped
// addresses and use zero constants (exact zero weights).  The slab constants
// are loaded first, the weight prefetch issued behind them, and only then
// staged to LDS.  All 64 * WAVES threads must call it (contains barriers).
template <int BITS, int MB, int NS>
struct SkinnyGeom {
  const uint32_t* wrow[NS];
  const uint16_t* xr[MB];
  const f32x4* gcol[NS];
  int u0, nu, nsteps, chunks, g, gs_shift;
  bool col_ok[NS];
  __device__ __forceinline__ int chunk_of(int j) const { return min(4 * (u0 + j) + g, chunks - 1); }
  __device__ __forceinline__ void load_x(int j, u32x4 (&dst)[MB][4]) const {
    const int c = chunk_of(j);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[mb][i] = u32x4{0u, 0u, 0u, 0u};
      if (xr[mb]) {
        const u32x4* xs = reinterpret_cast<const u32x4*>(xr[mb] + (size_t)c * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[mb][i] = xs[i];
      }
    }
  }
};

// NS slabs (16 columns each) share every activation slice a step loads.
template <typename TT, int BITS, int MB, bool FAST, int PF, int NS>
__device__ __forceinline__ void skinny_stream(const SkinnyGeom<BITS, MB, NS>& sg, uint32_t (&wbuf)[NS][PF][BITS],
                                              u32x4 (&xa)[2][MB][4], f32x4 (&acc)[NS][MB]) {
  for (int base = 0; base < sg.nsteps; base += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int j = base + p;
      uint32_t cur[NS][BITS];
#pragma unroll
      for (int sl = 0; sl < NS; ++sl)
#pragma unroll
        for (int i = 0; i < BITS; ++i) cur[sl][i] = wbuf[sl][p][i];
      if (base + PF < sg.nsteps)
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) load_chunk<BITS>(sg.wrow[sl], (size_t)sg.chunk_of(j + PF), wbuf[sl][p]);
      if (j + 1 < sg.nsteps) sg.load_x(j + 1, xa[(p + 1) & 1]);
      const int c = 4 * (sg.u0 + j) + sg.g;
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        f32x4 gcv = sg.gcol[sl][(min(c, sg.chunks - 1) << 5) >> sg.gs_shift];
        if (j >= sg.nu || c >= sg.chunks || !sg.col_ok[sl]) gcv = f32x4{0.f, 0.f, 0.f, 0.f};
        const float sf = gcv[0], bf = gcv[1], s16 = sf * 0.0625f;
        u32x4 bop[4];
        bop[0] = dequant_slice_nat<TT, BITS, FAST, 0>(cur[sl], sf, s16, bf, gcv[2], gcv[3]);
        bop[1] = dequant_slice_nat<TT, BITS, FAST, 1>(cur[sl], sf, s16, bf, gcv[2], gcv[3]);
        bop[2] = dequant_slice_nat<TT, BITS, FAST, 2>(cur[sl], sf, s16, bf, gcv[2], gcv[3]);
        bop[3] = dequant_slice_nat<TT, BITS, FAST, 3>(cur[sl], sf, s16, bf, gcv[2], gcv[3]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[sl][mb] = Mfma16<TT>::run(xa[p & 1][mb][i], bop[i], acc[sl][mb]);
      }
    }
  }
}

template <typename TT, int BITS, int MB, int WAVES, class SH, int NS = 1>
__device__ __forceinline__ void skinny_tile(const uint32_t* __restrict__ w,
                                            const uint16_t* __restrict__ scales,
                                            const uint16_t* __restrict__ biases, int n, int k,
                                            int gs_shift, int n0, f32x4* gc, SH& sh) {
  constexpr int PF = 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int G = k >> gs_shift, GP = G + 1;
  const bool vec = (G & 7) == 0 &&
                   ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases)) & 15u) == 0;

  SkinnyGeom<BITS, MB, NS> sg;
  sg.chunks = k >> 5;
  const int units = (sg.chunks + 3) >> 2;
  const int per = (units + WAVES - 1) / WAVES;
  sg.u0 = wave * per;
  sg.nu = min(units, sg.u0 + per) - sg.u0;
  sg.nsteps = (max(sg.nu, 0) + PF - 1) / PF * PF;
  sg.g = lane >> 4;
  sg.gs_shift = gs_shift;
#pragma unroll
  for (int sl = 0; sl < NS; ++sl) {
    const int col = n0 + 16 * sl + nl;
    sg.col_ok[sl] = col < n;
    sg.wrow[sl] = w + (size_t)(sg.col_ok[sl] ? col : 0) * ((size_t)k * BITS / 32);
    sg.gcol[sl] = gc + (16 * sl + nl) * GP;
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) sg.xr[mb] = sh.xrow[16 * mb + nl];

  // 1. Constants' loads, then the weight / activation prefetch behind them.
  SlabConsts sc[NS];
#pragma unroll
  for (int sl = 0; sl < NS; ++sl) slab_consts_load<64 * WAVES>(scales, biases, n, G, n0 + 16 * sl, vec, sc[sl]);
  uint32_t wbuf[NS][PF][BITS];
  u32x4 xa[2][MB][4];
  if (sg.nsteps > 0) {
#pragma unroll
    for (int p = 0; p < PF; ++p)
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) load_chunk<BITS>(sg.wrow[sl], (size_t)sg.chunk_of(p), wbuf[sl][p]);
    sg.load_x(0, xa[0]);
  }
  // 2. Constants into LDS, vote (slab 16 sl + c at gc[(16 sl + c) * GP + g]).
  bool fast = true;
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
    fast &= slab_consts_store<TT, 64 * WAVES>(scales, biases, n, G, n0 + 16 * sl, vec, sc[sl], gc + 16 * sl * GP, GP);

  // 3. Stream.
  f32x4 acc[NS][MB];
#pragma unroll
  for (int sl = 0; sl < NS; ++sl)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[sl][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (sg.nsteps > 0) {
    if constexpr (BITS == 4 || BITS == 8) {
      if (fast)
        skinny_stream<TT, BITS, MB, true, PF, NS>(sg, wbuf, xa, acc);
      else
        skinny_stream<TT, BITS, MB, false, PF, NS>(sg, wbuf, xa, acc);
    } else {
      skinny_stream<TT, BITS, MB, false, PF, NS>(sg, wbuf, xa, acc);
    }
  }

  // 4. Sum the K-partial tiles, one slab at a time.
#pragma unroll
  for (int sl = 0; sl < NS; ++sl) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sh.red[wave][mb][lane][i] = acc[sl][mb][i];
    }
    __syncthreads();
    // Each wave finishes MB/4 (at least one) of the 16-row blocks.
    const int col = n0 + 16 * sl + nl;
    for (int mb = wave; mb < MB; mb += WAVES) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = sh.red[0][mb][lane][i];
#pragma unroll
        for (int wv = 1; wv < WAVES; ++wv) v += sh.red[wv][mb][lane][i];
        const int m = 16 * mb + 4 * sg.g + i;  // D row of element i in this lane
        uint16_t* yr = sh.yrow[m];
        if (yr && sg.col_ok[sl]) yr[col] = TT::from_f32(v);
      }
    }
    __syncthreads();
  }
}

template <typename TT, int BITS, int MB, int WAVES, int NS = 1>
__global__ __launch_bounds__(64 * WAVES) void skinny_kernel(const uint32_t* __restrict__ w,
                                                     const uint16_t* __restrict__ scales,
                                                     const uint16_t* __restrict__ biases,
                                                     const uint16_t* __restrict__ x,
                                                     uint16_t* __restrict__ y, int m, int n, int k,
                                                     int gs_shift) {
  __shared__ TileShared<WAVES, MB> sh;
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  f32x4* gc = reinterpret_cast<f32x4*>(dyn);
  const int n0 = blockIdx.x * 16 * NS;
  const int row0 = blockIdx.y * 16 * MB;
  if (threadIdx.x < 16 * MB) {
    const int r = row0 + threadIdx.x;
    sh.xrow[threadIdx.x] = r < m ? x + (size_t)r * k : nullptr;
    sh.yrow[threadIdx.x] = r < m ? y + (size_t)r * n : nullptr;
  }
  __syncthreads();
  skinny_tile<TT, BITS, MB, WAVES, TileShared<WAVES, MB>, NS>(w, scales, biases, n, k, gs_shift, n0, gc, sh);
}

// Routed experts: workgroup (16-column slab, expert e).  Rows routed to e are
// gathered 64 at a time (ballot compaction over rhs, or a binary-searched run
// when rhs is sorted), then run through skinny_tile against W[e].  Rows whose
// lhs index is out of range are skipped here and zeroed by gather_check_kernel.
template <typename TT, int BITS>
__global__ __launch_bounds__(256) void gather_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, int x_rows,
    const uint32_t* __restrict__ lhs, const uint32_t* __restrict__ rhs, int n_rows,
    uint16_t* __restrict__ y, int n, int k, int gs_shift, int sorted) {
  __shared__ TileShared<4, kMaxMB> sh;
  extern __shared__ __attribute__((aligned(16))) unsigned char dyn[];
  f32x4* gc = reinterpret_cast<f32x4*>(dyn);
  const int n0 = blockIdx.x * 16;
  const uint32_t e = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t expert_words = (size_t)n * k * BITS / 32;
  const size_t expert_groups = (size_t)n * (k >> gs_shift);
  const uint32_t* we = w + e * expert_words;
  const uint16_t* se = scales + e * expert_groups;
  const uint16_t* be = biases + e * expert_groups;

  int lo = 0, hi = n_rows;
  if (sorted) {
    // [lo, hi) = equal range of e in the ascending rhs (gather_qmm_rhs walks
    // these runs, quantized.h:2329-2345).
    int a = 0, b = n_rows;
    while (a < b) { int mid = (a + b) >> 1; if (rhs[mid] < e) a = mid + 1; else b = mid; }
    lo = a;
    b = n_rows;
    while (a < b) { int mid = (a + b) >> 1; if (rhs[mid] <= e) a = mid + 1; else b = mid; }
    hi = a;
  }
  if (threadIdx.x == 0) sh.pos = lo;
  __syncthreads();

  while (true) {
    const int pos = sh.pos;
    // Every wave has read pos before wave 0 overwrites it below, so all waves
    // agree on the trip count (and on every barrier).
    __syncthreads();
    if (pos >= hi) break;
    if (wave == 0) {
      int p = pos, cnt = 0;
      if (sorted) {
        cnt = min(64, hi - p);
        if (lane < cnt) sh.rows[lane] = p + lane;
        p += cnt;
      } else {
        while (p < hi && cnt < 64) {
          const int r = p + lane;
          const bool match = r < hi && rhs[r] == e;
          const unsigned long long mask = __ballot(match);
          const int rank = __popcll(mask & ((1ull << lane) - 1ull));
          const bool take = match && (cnt + rank < 64);
          if (take) sh.rows[cnt + rank] = r;
          const unsigned long long left = mask & ~__ballot(take);
          const int took = __popcll(mask) - __popcll(left);
          cnt += took;
          p = left ? p + (int)__ffsll((long long)left) - 1 : p + 64;
        }
      }
      if (lane == 0) {
        sh.count = cnt;
        sh.pos = p;
      }
    }
    __syncthreads();
    const int cnt = sh.count;
    if (threadIdx.x < 64) {
      const int i = threadIdx.x;
      const uint16_t* xp = nullptr;
      uint16_t* yp = nullptr;
      if (i < cnt) {
        const int r = sh.rows[i];
        const uint32_t xi = lhs ? lhs[r] : (uint32_t)r;
        if (xi < (uint32_t)x_rows) {
          xp = x + (size_t)xi * k;
          yp = y + (size_t)r * n;
        }
      }
      sh.xrow[i] = xp;
      sh.yrow[i] = yp;
    }
    __syncthreads();
    if (cnt == 0) continue;  // uniform: the scan reached hi without a match
    if (cnt <= 16) {
      skinny_tile<TT, BITS, 1, 4>(we, se, be, n, k, gs_shift, n0, gc, sh);
    } else if (cnt <= 32) {
      skinny_tile<TT, BITS, 2, 4>(we, se, be, n, k, gs_shift, n0, gc, sh);
    } else {
      skinny_tile<TT, BITS, 4, 4>(we, se, be, n, k, gs_shift, n0, gc, sh);
    }
  }
}

// Validates routing indices on the device: out-of-range rows are zeroed and
// counted; with sorted=1 every descent is counted too.
template <typename TT>
__global__ __launch_bounds__(256) void gather_check_kernel(const uint32_t* __restrict__ lhs,
                                                           const uint32_t* __restrict__ rhs,
                                                           int n_rows, int x_rows, int n_experts,
                                                           int sorted, uint16_t* __restrict__ y,
                                                           int n, unsigned int* status) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_rows) return;
  const bool bad = rhs[r] >= (uint32_t)n_experts || (lhs && lhs[r] >= (uint32_t)x_rows);
  const bool unsorted = sorted && r + 1 < n_rows && rhs[r] > rhs[r + 1];
  if (bad) {
    for (int j = 0; j < n; ++j) y[(size_t)r * n + j] = 0;
  }
  if (bad || unsorted) atomicAdd(status, 1u);
}

int shift_of(int gs) {
  int s = 0;
  while ((1 << s) < gs) ++s;
  return s;
}

// Dynamic LDS of the slab constants: 16 columns x (K/gs + 1) f32x4.
size_t slab_consts_bytes(int k, int gs) { return (size_t)16 * (k / gs + 1) * 16; }

// Raises the kernel's dynamic-LDS limit to what the CU holds (once per kernel).
template <typename TT, int BITS, int MB, int WAVES, int NS>
hipError_t skinny_allow_lds() {
  static const hipError_t e = [] {
    const void* fn = reinterpret_cast<const void*>(&skinny_kernel<TT, BITS, MB, WAVES, NS>);
    hipFuncAttributes fa;
    hipError_t r = hipFuncGetAttributes(&fa, fn);
    if (r != hipSuccess) return r;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(160 * 1024 - fa.sharedSizeBytes));
  }();
  return e;
}

template <typename TT, int BITS>
hipError_t launch_skinny_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                           int k) {
  const int gs_shift = shift_of(q.gs);
  const int mb = (m + 15) / 16;
  const auto* sc = static_cast<const uint16_t*>(q.scales);
  const auto* bi = static_cast<const uint16_t*>(q.biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  const unsigned gx = (unsigned)((n + 15) / 16);
  const unsigned gy = mb <= 2 ? 1u : (unsigned)((m + 63) / 64);
  const size_t lds = slab_consts_bytes(k, q.gs);
  // Few slabs (under two per CU): 8 waves per workgroup keep two waves per
  // SIMD streaming; otherwise 4.
  static const int forced = env_int("CPQ_SKINNY_WAVES", 0);
  const bool eight = forced ? forced == 8 : (size_t)gx * gy < 512;
  // Slab constants past the default 64 KiB of dynamic LDS (long K, small
  // groups) need the kernel's limit raised first.
  auto go = [&](auto kern, int waves, hipError_t (*allow)()) -> hipError_t {
    if (lds > (size_t)64 * 1024) {
      const hipError_t a = allow();
      if (a != hipSuccess) return a;
    }
    hipLaunchKernelGGL(kern, dim3(gx, gy), dim3(64 * waves), lds, s, q.w, sc, bi, xx, yy, m, n, k, gs_shift);
    return hipGetLastError();
  };
  if (mb <= 1) {
    return eight ? go(skinny_kernel<TT, BITS, 1, 8>, 8, &skinny_allow_lds<TT, BITS, 1, 8, 1>)
                 : go(skinny_kernel<TT, BITS, 1, 4>, 4, &skinny_allow_lds<TT, BITS, 1, 4, 1>);
  } else if (mb <= 2) {
    return eight ? go(skinny_kernel<TT, BITS, 2, 8>, 8, &skinny_allow_lds<TT, BITS, 2, 8, 1>)
                 : go(skinny_kernel<TT, BITS, 2, 4>, 4, &skinny_allow_lds<TT, BITS, 2, 4, 1>);
  } else {
    // 64 activation rows: the activation slices dominate the L2 traffic (every
    // slab rereads all of X), so once two-slab workgroups still give every
    // CU one (N >= 32 x CUs) a workgroup takes two slabs per activation load
    // (M = 64, N = 8192: 38.0 -> 23.4 us; at N = 4096 half the CUs would
    // idle: 19.3 vs 22.2 us).  4 waves measure faster than 8.
    static const int two_slabs = env_int("CPQ_SKINNY_NS", 0);  // tuning hook: 1 or 2 slabs per workgroup
    static const int cus = [] {
      int dev = 0, cu = 0;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
        cu = 256;
      return cu;
    }();
    const bool ns2 = two_slabs ? two_slabs == 2 : (n + 31) / 32 >= cus;
    if (ns2 && 2 * lds + sizeof(TileShared<4, 4>) <= (size_t)160 * 1024) {
      const hipError_t a = skinny_allow_lds<TT, BITS, 4, 4, 2>();
      if (a != hipSuccess) return a;
      hipLaunchKernelGGL((skinny_kernel<TT, BITS, 4, 4, 2>), dim3((unsigned)((n + 31) / 32), gy), dim3(256), 2 * lds,
                         s, q.w, sc, bi, xx, yy, m, n, k, gs_shift);
    } else {
      return go(skinny_kernel<TT, BITS, 4, 4>, 4, &skinny_allow_lds<TT, BITS, 4, 4, 1>);
    }
  }
  return hipGetLastError();
}

template <typename TT, int BITS>
hipError_t launch_gather_t(hipStream_t s, const QuantArgs& q, const void* x, int x_rows,
                           const uint32_t* lhs, const uint32_t* rhs, int n_rows, void* y,
                           int n_experts, int n, int k, bool sorted, unsigned int* status) {
  if (n_rows == 0) return hipSuccess;
  const int gs_shift = shift_of(q.gs);
  // Few rows (decode): one pass per distinct expert (validates the indices itself).
  if (gather_decode_supported(q, x_rows, n_rows, n, k))
    return launch_gather_decode(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, status);
  if (gather_expert_supported(BITS, x_rows, n_rows, n, k)) {  // validates the indices itself
    static const int cus = [] {
      int dev = 0, cu = 0;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
        cu = 256;
      return cu;
    }();
    return launch_gather_expert(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, cus, status);
  }
  // The shape must fit before anything is enqueued (the check kernel below
  // writes y and the status word).
  const size_t lds = slab_consts_bytes(k, q.gs);
  if (lds + sizeof(TileShared<4, kMaxMB>) > (size_t)160 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gather_check_kernel<TT>), dim3((n_rows + 255) / 256), dim3(256), 0, s, lhs,
                     rhs, n_rows, x_rows, n_experts, (int)sorted, static_cast<uint16_t*>(y), n,
                     status);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (lds > (size_t)64 * 1024) {  // long K, small groups: raise the kernel's dynamic-LDS limit once
    static const hipError_t a = [] {
      const void* fn = reinterpret_cast<const void*>(&gather_kernel<TT, BITS>);
      hipFuncAttributes fa;
      hipError_t r = hipFuncGetAttributes(&fa, fn);
      if (r != hipSuccess) return r;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (a != hipSuccess) return a;
  }
  hipLaunchKernelGGL((gather_kernel<TT, BITS>), dim3((unsigned)((n + 15) / 16), (unsigned)n_experts),
                     dim3(256), lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     x_rows, lhs, rhs, n_rows, static_cast<uint16_t*>(y), n, k, gs_shift,
                     (int)sorted);
  return hipGetLastError();
}

#define CPQ_BITS_SWITCH(FN, TT, ...)                 \
  switch (q.bits) {                                  \
    case 2: return FN<TT, 2>(__VA_ARGS__);           \
    case 3: return FN<TT, 3>(__VA_ARGS__);           \
    case 4: return FN<TT, 4>(__VA_ARGS__);           \
    case 5: return FN<TT, 5>(__VA_ARGS__);           \
    case 6: return FN<TT, 6>(__VA_ARGS__);           \
    case 8: return FN<TT, 8>(__VA_ARGS__);           \
    default: return hipErrorInvalidValue;            \
  }

}  // namespace

bool skinny_fits(int k, int gs) {
  return gs > 0 && slab_consts_bytes(k, gs) + sizeof(TileShared<8, kMaxMB>) <= (size_t)160 * 1024;
}

bool gather_supported(int bits, int n_rows, int n, int k, int gs) {
  const QuantArgs shape{nullptr, nullptr, nullptr, gs, bits, CPQ_DTYPE_BF16};
  return gather_decode_supported(shape, 1, n_rows, n, k) ||
         gather_expert_supported(bits, 1, n_rows, n, k) ||
         (gs > 0 && slab_consts_bytes(k, gs) + sizeof(TileShared<4, kMaxMB>) <= (size_t)160 * 1024);
}

hipError_t launch_qmm_skinny(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m,
                             int n, int k) {
  if (q.dtype == CPQ_DTYPE_BF16) { CPQ_BITS_SWITCH(launch_skinny_t, BF16, s, q, x, y, m, n, k) }
  if (q.dtype == CPQ_DTYPE_F16) { CPQ_BITS_SWITCH(launch_skinny_t, F16, s, q, x, y, m, n, k) }
  return hipErrorInvalidValue;
}

hipError_t launch_gather_qmm(hipStream_t s, const QuantArgs& q, const void* x, int x_rows,
                             const uint32_t* lhs, const uint32_t* rhs, int n_rows, void* y,
                             int n_experts, int n, int k, bool sorted, unsigned int* status) {
  if (q.dtype == CPQ_DTYPE_BF16) {
    CPQ_BITS_SWITCH(launch_gather_t, BF16, s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k,
                    sorted, status)
  }
  if (q.dtype == CPQ_DTYPE_F16) {
    CPQ_BITS_SWITCH(launch_gather_t, F16, s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k,
                    sorted, status)
  }
  return hipErrorInvalidValue;
}

}  // namespace cpq
