// Decode GEMV (M = 1) for gfx950: y[n] = sum_k x[k] * RNE_T(fmaf(s, q[n,k], b)).
//
// Reference op: affine_qmv_fast / affine_qmv (kernels-mlx/.../quantized.h:749-975),
// dispatched by crates/cider-press-kernels/src/kernels/qmv.rs:77-205.
// Numerics follow the dequantize-then-dot contract (weights rounded to T,
// fp32 accumulation) rather than MLX's unrounded factored form: with bf16
// outputs the factored form exceeds the 2e-3 relative-L2 budget at K=4096.
//
// HBM-bound: algorithmic bytes per call = N*K*bits/8 + 2*N*(K/gs)*sizeof(T)
// + (K + N)*sizeof(T).  Per weight the only real work is the VALU
// dequantization, so the dot products go to the matrix cores:
//   - a workgroup owns 16 output rows and gives each of its WAVES waves a
//     contiguous quarter (eighth) of K;
//   - loads are issued in the order they are needed: first the 16 rows'
//     scales and biases and the activation (small), then the first PF weight
//     chunks of every lane; the small loads return first, are staged into LDS
//     (activation permuted into the dequantizer's interleaved slot order,
//     per-group constants s, b, b-1024s, b-64s precomputed) and a workgroup
//     vote picks the single-FMA fast dequantization when it is exact for
//     every group, while the weight stream is already in flight;
//   - lane l streams row n0 + l%16, chunk 4u + l/16 (16 B at 4-bit: each wave
//     instruction reads 64 contiguous bytes of 16 rows, consecutive steps the
//     next 64), PF chunks in flight;
//   - each 8-element slice is dequantized into an MFMA B operand and issued
//     as v_mfma_f32_16x16x32 against the activation slice broadcast to all 16
//     A rows (the matrix cores are otherwise idle at M = 1);
//   - the K-partial results of the waves are summed through LDS.
#include <algorithm>
#include <type_traits>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

struct QmvGeom {
  const uint32_t* wrow;
  const uint16_t* xs;
  const f32x4* gcrow;  // per-group (s, b, c0, c1) of this lane's row
  int chunks, gs_shift, g;
  int u0, u_end;       // this wave's unit range [u0, u_end)
};

// Chunk of step j (clamped to a valid chunk so loads never leave the row).
template <bool EXACT>
__device__ __forceinline__ int chunk_at(const QmvGeom& q, int j) {
  const int c = 4 * (q.u0 + j) + q.g;
  if constexpr (EXACT) return c;
  return min(c, q.chunks - 1);
}

template <int BITS, bool EXACT>
__device__ __forceinline__ void fetch(const QmvGeom& q, int j, uint32_t* dst) {
  load_chunk<BITS>(q.wrow, (size_t)chunk_at<EXACT>(q, j), dst);
}

// One K step: 32 weights of this lane's row, 4 MFMAs.  In the inexact
// geometry, steps past this wave's range use zero constants (exact zeros).
template <typename TT, int BITS, bool EXACT, bool FAST>
__device__ __forceinline__ void step(const QmvGeom& q, const uint32_t* cur, int j, f32x4& acc) {
  const int c = chunk_at<EXACT>(q, j);
  f32x4 gc = q.gcrow[(c << 5) >> q.gs_shift];
  if constexpr (!EXACT) {
    const bool live = q.u0 + j < q.u_end && 4 * (q.u0 + j) + q.g < q.chunks;
    if (!live) gc = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float s = gc[0], b = gc[1], c0 = gc[2], c1 = gc[3];
  const float s16 = s * 0.0625f;
  const u32x4* xa = reinterpret_cast<const u32x4*>(q.xs + c * 32);
  acc = Mfma16<TT>::run(xa[0], dequant_slice<TT, BITS, FAST, 0>(cur, s, s16, b, c0, c1), acc);
  acc = Mfma16<TT>::run(xa[1], dequant_slice<TT, BITS, FAST, 1>(cur, s, s16, b, c0, c1), acc);
  acc = Mfma16<TT>::run(xa[2], dequant_slice<TT, BITS, FAST, 2>(cur, s, s16, b, c0, c1), acc);
  acc = Mfma16<TT>::run(xa[3], dequant_slice<TT, BITS, FAST, 3>(cur, s, s16, b, c0, c1), acc);
}

// Steady state keeps PF loads in flight (loads unconditional, buffer index
// static after unrolling), then drains the last PF steps.
template <typename TT, int BITS, int PF, bool EXACT, bool FAST>
__device__ __forceinline__ f32x4 stream(const QmvGeom& q, int nsteps, uint32_t (&buf)[PF][BITS]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int base = 0; base < nsteps - PF; base += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      uint32_t cur[BITS];
#pragma unroll
      for (int i = 0; i < BITS; ++i) cur[i] = buf[p][i];
      fetch<BITS, EXACT>(q, base + PF + p, buf[p]);
      step<TT, BITS, EXACT, FAST>(q, cur, base + p, acc);
    }
  }
#pragma unroll
  for (int p = 0; p < PF; ++p) step<TT, BITS, EXACT, FAST>(q, buf[p], nsteps - PF + p, acc);
  return acc;
}

constexpr int kSegSlots = 2;  // 8-B scale/bias quads held per thread before the weight loads
constexpr int kXSlots = 4;    // 16-B activation slices held per thread before the weight loads

template <typename TT>
__device__ __forceinline__ f32x4 group_consts(uint32_t sv, uint32_t bv) {
  const float s = TT::to_f32((uint16_t)sv), b = TT::to_f32((uint16_t)bv);
  return f32x4{s, b, fmaf(-1024.f, s, b), fmaf(-64.f, s, b)};
}

// One chunk (BITS words) of a weight row through a buffer descriptor.
// One chunk of a lane's weight stream (16 bytes at 4 bits, 32 at 8).  NT
// sets the non-temporal policy (streamed once; the weights need not stay in
// the caches).  Measured on the 4-bit decode layout with M rows: M = 4 /
// 16 at N = K = 4096 4.85 -> 4.46 / 6.11 -> 5.95 us on two boxes.  The
// M = 1 decode kernel at cfg2a moved by -0.17 us on one box and +0.19 us on
// another, and cfg2b, cfg1 and the 8-bit step-interleaved rows were slower
// with it, so they keep the default policy.
template <int BITS, bool NT>
__device__ __forceinline__ void lean_load_nt(__amdgpu_buffer_rsrc_t wr, uint32_t voff, int soff, uint32_t* dst) {
  constexpr int POL = NT ? 2 : 0;  // cache policy: nt
  if constexpr (BITS == 4) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, soff, POL));
    dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
  } else {
    const u32x4 v0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, soff, POL));
    const u32x4 v1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff + 16, soff, POL));
    dst[0] = v0.x; dst[1] = v0.y; dst[2] = v0.z; dst[3] = v0.w;
    dst[4] = v1.x; dst[5] = v1.y; dst[6] = v1.z; dst[7] = v1.w;
  }
}

template <int BITS>
__device__ __forceinline__ void lean_load(__amdgpu_buffer_rsrc_t wr, uint32_t voff, int soff, uint32_t* dst) {
  lean_load_nt<BITS, false>(wr, voff, soff, dst);
}

template <typename TT, int BITS, int WAVES, int PF, bool EXACT>
__global__ __launch_bounds__(64 * WAVES) void qmv_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int n, int k,
                                                         int gs_shift) {
  constexpr int NT = 64 * WAVES;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int G = k >> gs_shift;
  const int GP = G + 1;  // padded row stride: the 16 rows of a lane group hit distinct banks
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);                          // k, interleaved
  f32x4* gct = reinterpret_cast<f32x4*>(smem + (size_t)k * 2);                 // [16][GP]
  float* red = reinterpret_cast<float*>(smem + (size_t)k * 2 + (size_t)16 * GP * 16);  // [WAVES][16]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15;
  const int n0 = blockIdx.x * 16;
  const int row = n0 + nl;
  const int chunks = k >> 5;
  const int units = (chunks + 3) >> 2;
  const int per_wave = (units + WAVES - 1) / WAVES;

  QmvGeom q;
  q.wrow = w + (size_t)(row < n ? row : 0) * ((size_t)k * BITS / 32);
  q.xs = xs;
  q.gcrow = gct + nl * GP;
  q.chunks = chunks;
  q.gs_shift = gs_shift;
  q.g = lane >> 4;
  q.u0 = wave * per_wave;
  q.u_end = min(units, q.u0 + per_wave);
  const int nsteps = (per_wave + PF - 1) / PF * PF;

  // 1. Small loads first: (scale, bias) quads (4 groups, 8 B) of the 16 rows,
  //    then the activation.
  const bool vec = (G & 3) == 0 &&
                   ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases)) & 7u) == 0;
  const int quads = G >> 2;
  u32x2 sv[kSegSlots], bv[kSegSlots];
#pragma unroll
  for (int t = 0; t < kSegSlots; ++t) {
    const int i = tid + t * NT;
    sv[t] = bv[t] = u32x2{0u, 0u};
    if (vec && i < 16 * quads) {
      const int r = i / quads, sg = i - r * quads;
      if (n0 + r < n) {
        sv[t] = *reinterpret_cast<const u32x2*>(scales + (size_t)(n0 + r) * G + sg * 4);
        bv[t] = *reinterpret_cast<const u32x2*>(biases + (size_t)(n0 + r) * G + sg * 4);
      }
    }
  }
  u32x4 xv[kXSlots];
#pragma unroll
  for (int t = 0; t < kXSlots; ++t) {
    const int i = tid + t * NT;
    xv[t] = u32x4{0u, 0u, 0u, 0u};
    if (i < (k >> 3)) xv[t] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
  }

  // 2. The weight stream.
  uint32_t buf[PF][BITS];
#pragma unroll
  for (int p = 0; p < PF; ++p) fetch<BITS, EXACT>(q, p, buf[p]);

  // 3. Stage to LDS (and anything beyond the register slots), vote: one
  //    packed check over all of this thread's groups, the exact per-group
  //    predicate only where the packed check fails (zero scales or biases).
#pragma unroll
  for (int t = 0; t < kXSlots; ++t) {
    const int i = tid + t * NT;
    if (i < (k >> 3)) *reinterpret_cast<u32x4*>(xs + (size_t)i * 8) = interleave_x<BITS>(xv[t]);
  }
  for (int i = tid + kXSlots * NT; i < (k >> 3); i += NT) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    *reinterpret_cast<u32x4*>(xs + (size_t)i * 8) = interleave_x<BITS>(v);
  }
  bool ok = true;
  if (vec) {
    FastQuick fq;
    fast_quick_init(fq);
#pragma unroll
    for (int t = 0; t < kSegSlots; ++t) {
      const int i = tid + t * NT;
      if (i < 16 * quads) {
        const int r = i / quads, sg = i - r * quads;
        f32x4* dst = gct + r * GP + sg * 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t s2 = sv[t][h], b2 = bv[t][h];
          dst[2 * h] = group_consts<TT>(s2 & 0xffffu, b2 & 0xffffu);
          dst[2 * h + 1] = group_consts<TT>(s2 >> 16, b2 >> 16);
          fast_quick_add<TT>(fq, s2, b2);
        }
      }
    }
    if (!fast_quick_ok<TT>(fq)) {
#pragma unroll
      for (int t = 0; t < kSegSlots; ++t) {
        if (tid + t * NT < 16 * quads) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            ok &= fast_ok_bits<TT>(sv[t][h] & 0xffffu, bv[t][h] & 0xffffu) &
                  fast_ok_bits<TT>(sv[t][h] >> 16, bv[t][h] >> 16);
        }
      }
    }
    for (int i = tid + kSegSlots * NT; i < 16 * quads; i += NT) {
      const int r = i / quads, sg = i - r * quads;
      u32x2 s4 = {0u, 0u}, b4 = {0u, 0u};
      if (n0 + r < n) {
        s4 = *reinterpret_cast<const u32x2*>(scales + (size_t)(n0 + r) * G + sg * 4);
        b4 = *reinterpret_cast<const u32x2*>(biases + (size_t)(n0 + r) * G + sg * 4);
      }
      f32x4* dst = gct + r * GP + sg * 4;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        dst[2 * h] = group_consts<TT>(s4[h] & 0xffffu, b4[h] & 0xffffu);
        dst[2 * h + 1] = group_consts<TT>(s4[h] >> 16, b4[h] >> 16);
        ok &= fast_ok_bits<TT>(s4[h] & 0xffffu, b4[h] & 0xffffu) & fast_ok_bits<TT>(s4[h] >> 16, b4[h] >> 16);
      }
    }
  } else {
    for (int i = tid; i < 16 * G; i += NT) {
      const int r = i / G, gi = i - r * G;
      uint32_t s1 = 0, b1 = 0;
      if (n0 + r < n) {
        s1 = scales[(size_t)(n0 + r) * G + gi];
        b1 = biases[(size_t)(n0 + r) * G + gi];
      }
      gct[r * GP + gi] = group_consts<TT>(s1, b1);
      ok &= fast_ok_bits<TT>(s1, b1);
    }
  }
  const bool fast = __syncthreads_and(ok);

  // 4. Stream the weights.
  const f32x4 acc = fast ? stream<TT, BITS, PF, EXACT, true>(q, nsteps, buf)
                         : stream<TT, BITS, PF, EXACT, false>(q, nsteps, buf);

  // D[m][n] sits in lane n + 16*(m/4), element m%4; every A row holds x, so
  // lanes 0..15 element 0 carry row n0 + lane.
  if (lane < 16) red[wave * 16 + lane] = acc[0];
  __syncthreads();
  if (tid < 16 && n0 + tid < n) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) v += red[i * 16 + tid];
    y[n0 + tid] = TT::from_f32(v);
  }
}

// ---------------------------------------------------------------------------
// Lean decode kernel (4/8-bit, K % 2048 == 0, gs in {32, 64, 128}).
//
// Same work split as qmv_kernel (16 rows per workgroup, K split over 4 waves,
// lane = (row l%16, chunk 4u + l/16)), but every wave is self-contained until
// the final sum, and its fixed work is cut to a few dozen instructions so the
// VALU time goes to dequantization:
//   - a wave loads and stages only what its own K range needs (its 16 x 16B
//     activation items per step batch, the constants of its own groups) into
//     a private LDS region, votes for the fast path within the wave, and
//     starts streaming without waiting for the other waves;
//   - every global access is a buffer load: per-step offsets are immediates
//     or one scalar, rows past N read zeros (range-checked by the
//     descriptor), so there are no per-load address computations and no
//     bounds branches;
//   - the group constants and activation slices of step j sit at immediate
//     LDS offsets from one per-lane base (gs is a template parameter).
// ---------------------------------------------------------------------------
constexpr int kLeanXItems = 8;   // 16-B activation items per lane (K <= 16384)
constexpr int kLeanQuads = 8;    // 8-B scale/bias quads per lane (wave's groups per row <= 128)

// Per-wave LDS: activations (256 B per step and row) then constants [16][GW + 1].
__host__ __device__ constexpr size_t lean_wave_lds(int nsteps, int gs_shift, int rows = 1, int cw = 16) {
  return (size_t)256 * nsteps * rows + (size_t)16 * ((size_t)nsteps * (128 >> gs_shift) + 1) * cw;
}

// MR > 1: xbase holds the lane's slice-0 address; slice i of step j sits at
// xbase + xsw[i] + j * STEP_X (per-lane swizzled offsets of its row).
// CW: bytes per group's constants, 16 (s, b, b - 1024 s, b - 64 s) or 8
// (s, b; the other two computed per step, the same fmaf).
struct NoStage {
  __device__ void operator()(int) const {}
};

// stage(j), where given, writes step j's activation slices into LDS (and
// orders them within the wave) right before the step's operands are read:
// the fully unrolled form then waits for each step's activations as it
// reaches them.
template <typename TT, int BITS, int GS_SHIFT, int PF, bool ONE, bool FAST, int MR = 1, int CW = 16,
          typename Stage = NoStage>
__device__ __forceinline__ f32x4 lean_stream(__amdgpu_buffer_rsrc_t wr, uint32_t voff, int nsteps,
                                             const unsigned char* cbase, const unsigned char* xbase,
                                             uint32_t (&buf)[PF][BITS], const int* xsw = nullptr,
                                             Stage stage = Stage{}) {
  constexpr int CB = BITS * 4;             // bytes per 32-element chunk
  constexpr int STEP_W = 4 * CB;           // weight bytes a lane group advances per step
  constexpr int STEP_C = (128 >> GS_SHIFT) * CW;  // constants bytes per step
  constexpr int STEP_X = 4 * 64;           // activation bytes per step (4 chunks x 32 x 2 B)
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // ONE: a step's LDS operands (its group constants and four activation
  // slices) are read one step ahead, so their latency runs under the
  // previous step's dequantization instead of in front of this one's (the
  // looped form keeps them in the step: the look-ahead's registers would
  // spill there).
  using CV = std::conditional_t<CW == 16, f32x4, f32x2>;
  struct Ops {
    CV gc;
    u32x4 a[4];
  };
  auto load_ops = [&](int j, Ops& o) {
    o.gc = *reinterpret_cast<const CV*>(cbase + j * STEP_C);
    const unsigned char* xj = xbase + j * STEP_X;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o.a[i] = *reinterpret_cast<const u32x4*>(xj + (MR == 1 ? 16 * i : xsw[i]));
  };
  auto step = [&](const uint32_t* cur, const Ops& o) {
    float sc, b, c0, c1;
    sc = o.gc[0];
    b = o.gc[1];
    if constexpr (CW == 16) {
      c0 = o.gc[2];
      c1 = o.gc[3];
    } else {
      c0 = FAST ? fmaf(-1024.f, sc, b) : 0.f;
      c1 = FAST ? fmaf(-64.f, sc, b) : 0.f;
    }
    const float s16 = sc * 0.0625f;
    acc = Mfma16<TT>::run(o.a[0], dequant_slice<TT, BITS, FAST, 0>(cur, sc, s16, b, c0, c1), acc);
    acc = Mfma16<TT>::run(o.a[1], dequant_slice<TT, BITS, FAST, 1>(cur, sc, s16, b, c0, c1), acc);
    acc = Mfma16<TT>::run(o.a[2], dequant_slice<TT, BITS, FAST, 2>(cur, sc, s16, b, c0, c1), acc);
    acc = Mfma16<TT>::run(o.a[3], dequant_slice<TT, BITS, FAST, 3>(cur, sc, s16, b, c0, c1), acc);
  };
  Ops ops;
  int base = 0;
  // ONE: the whole range is the PF prefetched steps (no loop, buffers consumed in place).
  for (; !ONE && base + PF < nsteps; base += PF) {
    const int soff = (base + PF) * STEP_W;
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      uint32_t cur[BITS];
#pragma unroll
      for (int i = 0; i < BITS; ++i) cur[i] = buf[p][i];
      lean_load<BITS>(wr, voff + p * STEP_W, soff, buf[p]);
      load_ops(base + p, ops);
      step(cur, ops);
    }
  }
  if constexpr (ONE) {
    Ops ops, nxt;
    stage(0);
    load_ops(0, ops);
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      if (p + 1 < PF) {
        stage(p + 1);
        load_ops(p + 1, nxt);
      }
      step(buf[p], ops);
      ops = nxt;
    }
  } else {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      load_ops(base + p, ops);
      step(buf[p], ops);
    }
  }
  return acc;
}

// Batch element z's operands (the batch in grid dimension y): indices over
// the batch shape, innermost dimension last, times each operand's element
// strides; the output block of element z follows the z blocks before it.
template <typename W, typename S, typename X, typename Y>
__device__ __forceinline__ void batch_operands(const BatchArgs& ba, uint32_t z, W& w, S& scales, S& biases, X& x,
                                               Y& y, size_t y_block) {
  y += (size_t)z * y_block;
  long long o[4] = {0, 0, 0, 0};
#pragma unroll
  for (int d = kMaxBatchDims - 1; d >= 0; --d)
    if (d < ba.nd) {
      const uint32_t sh = (uint32_t)ba.shape[d];
      const long long i = (long long)(z % sh);
      z /= sh;
#pragma unroll
      for (int op = 0; op < 4; ++op) o[op] += i * ba.st[op][d];
    }
  w += o[0];
  scales += o[1];
  biases += o[2];
  x += o[3];
}

template <typename TT, int BITS, int GS_SHIFT, int WAVES, int PF, bool ONE, bool BATCH>
__global__ __launch_bounds__(64 * WAVES) void qmv_lean_kernel(const uint32_t* __restrict__ w,
                                                                   const uint16_t* __restrict__ scales,
                                                                   const uint16_t* __restrict__ biases,
                                                                   const uint16_t* __restrict__ x,
                                                                   uint16_t* __restrict__ y, int n, int k,
                                                                   const BatchArgs ba) {
  if constexpr (BATCH) batch_operands(ba, blockIdx.y, w, scales, biases, x, y, (size_t)n);
  constexpr int CB = BITS * 4;
  constexpr int GPS = 128 >> GS_SHIFT;  // groups per step (4 chunks of 32)
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int G = k >> GS_SHIFT;
  const int nsteps = ONE ? PF : k / (128 * WAVES);  // steps per wave: K / (32 * 4 * waves)
  const int GW = nsteps * GPS;          // groups of one row in this wave's K range
  const int quads = GW >> 2;            // 8-B quads of one row in this wave's K range
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int u0 = wave * nsteps;         // first step unit of this wave
  const uint32_t rowbytes = (uint32_t)k * BITS / 8;
  unsigned char* xw = smem + (size_t)wave * lean_wave_lds(nsteps, GS_SHIFT);
  f32x4* cw = reinterpret_cast<f32x4*>(xw + (size_t)256 * nsteps);  // [16][GW + 1]
  float* red = reinterpret_cast<float*>(smem + (size_t)WAVES * lean_wave_lds(nsteps, GS_SHIFT));

  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)scales, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)biases, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, k * 2, 0x00020000);

  // 1. Small loads first: this wave's scale / bias quads (row lane/4, quad
  //    lane%4 + 4t) and its activation items (lane + 64t of its range).
  const int cr = lane >> 2;
  const uint32_t coff = ((uint32_t)(n0 + cr) * (uint32_t)G + (uint32_t)(u0 * GPS + 4 * (lane & 3))) * 2u;
  u32x2 sv[kLeanQuads], bv[kLeanQuads];
#pragma unroll
  for (int t = 0; t < kLeanQuads; ++t) {
    sv[t] = bv[t] = u32x2{0u, 0u};
    if (4 * t < quads) {
      sv[t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, coff + 32u * t, 0, 0));
      bv[t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(br, coff + 32u * t, 0, 0));
    }
  }
  const int xitems = 4 * nsteps;  // 16-B items of this wave per 16 lanes... per lane: nsteps / 4
  const uint32_t xoff = (uint32_t)u0 * 256u + (uint32_t)lane * 16u;
  u32x4 xv[kLeanXItems];
#pragma unroll
  for (int t = 0; t < kLeanXItems; ++t) {
    xv[t] = u32x4{0u, 0u, 0u, 0u};
    if (4 * t < nsteps)
      xv[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + 1024u * t, 0, 0));
  }
  (void)xitems;

  // 2. The weight stream: lane (r, g) reads chunk 4(u0 + j) + g of row n0 + r.
  const uint32_t voff = (uint32_t)(n0 + r) * rowbytes + (uint32_t)(4 * u0 + g) * CB;
  uint32_t buf[PF][BITS];
#pragma unroll
  for (int p = 0; p < PF; ++p) lean_load<BITS>(wr, voff + p * 4 * CB, 0, buf[p]);

  // 3. Stage this wave's activations and constants, vote within the wave.
#pragma unroll
  for (int t = 0; t < kLeanXItems; ++t)
    if (4 * t < nsteps) *reinterpret_cast<u32x4*>(xw + lane * 16 + 1024 * t) = interleave_x<BITS>(xv[t]);
  FastQuick fq;
  fast_quick_init(fq);
  const int cwp = GW + 1;
#pragma unroll
  for (int t = 0; t < kLeanQuads; ++t) {
    const int cq = (lane & 3) + 4 * t;
    if (4 * t < quads && cq < quads) {
      f32x4* dst = cw + cr * cwp + cq * 4;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        dst[2 * h] = group_consts<TT>(sv[t][h] & 0xffffu, bv[t][h] & 0xffffu);
        dst[2 * h + 1] = group_consts<TT>(sv[t][h] >> 16, bv[t][h] >> 16);
        fast_quick_add<TT>(fq, sv[t][h], bv[t][h]);
      }
    }
  }
  bool ok = true;
  if (!fast_quick_ok<TT>(fq)) {
#pragma unroll
    for (int t = 0; t < kLeanQuads; ++t) {
      const int cq = (lane & 3) + 4 * t;
      if (4 * t < quads && cq < quads) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          ok &= fast_ok_bits<TT>(sv[t][h] & 0xffffu, bv[t][h] & 0xffffu) &
                fast_ok_bits<TT>(sv[t][h] >> 16, bv[t][h] >> 16);
      }
    }
  }
  // Lanes of one wave read each other's LDS writes: order them within the wave.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool fast = __builtin_amdgcn_ballot_w64(!ok) == 0;

  // 4. Stream.  Step j of this lane: constants of local group j*GPS + (32g >> GS_SHIFT),
  //    activation chunk 4j + g of the wave's range; both advance by fixed bytes per step.
  const unsigned char* cbase = reinterpret_cast<const unsigned char*>(cw + r * cwp + ((g * 32) >> GS_SHIFT));
  const unsigned char* xbase = xw + g * 64;
  const f32x4 acc = fast ? lean_stream<TT, BITS, GS_SHIFT, PF, ONE, true>(wr, voff, nsteps, cbase, xbase, buf)
                         : lean_stream<TT, BITS, GS_SHIFT, PF, ONE, false>(wr, voff, nsteps, cbase, xbase, buf);

  if (lane < 16) red[wave * 16 + lane] = acc[0];
  __syncthreads();
  if (tid < 16 && n0 + tid < n) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) v += red[i * 16 + tid];
    y[n0 + tid] = TT::from_f32(v);
  }
}

// Up to 16 activation rows on the lean kernel's layout: the same workgroup
// (16 output columns, WAVES waves over K, each wave self-contained until the
// final sum), but each wave stages M rows of its activation range, row r at
// r * 256 * nsteps bytes of its region with 16-byte slot s of a step stored
// at slot s ^ swz_key(r), so the 16 lanes one A-operand read serves together
// hit 16 distinct slots.  Rows
// past M are not read: their A rows only feed output rows that are never
// stored.  NST steps per wave (K = 128 * WAVES * NST); at most 16
// activation items per lane (M * NST <= 64).  CW: bytes of a group's
// constants in LDS (16, or 8 where the four-float form does not fit).
template <typename TT, int BITS, int GS_SHIFT, int WAVES, int NST, bool BATCH, int CW = 16>
__global__ __launch_bounds__(64 * WAVES) void qmm_lean_rows_kernel(const uint32_t* __restrict__ w,
                                                                    const uint16_t* __restrict__ scales,
                                                                    const uint16_t* __restrict__ biases,
                                                                    const uint16_t* __restrict__ x,
                                                                    uint16_t* __restrict__ y, int m, int n, int k,
                                                                    const BatchArgs ba) {
  if constexpr (BATCH) batch_operands(ba, blockIdx.y, w, scales, biases, x, y, (size_t)m * n);
  constexpr int CB = BITS * 4;
  constexpr int GPS = 128 >> GS_SHIFT;
  constexpr int XMAX = 16;             // activation items per lane
  constexpr int IPR = NST / 4;         // items per row and lane
  constexpr int PF = NST < 8 ? NST : 8;
  constexpr bool ONE = NST == PF;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int G = k >> GS_SHIFT;
  constexpr int nsteps = NST;
  const int GW = nsteps * GPS;
  const int quads = GW >> 2;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int u0 = wave * nsteps;
  const int rows = min(m, 16);
  const int RB = 256 * nsteps;  // bytes of one activation row in a wave's region
  const uint32_t rowbytes = (uint32_t)k * BITS / 8;
  const size_t wlds = lean_wave_lds(nsteps, GS_SHIFT, rows, CW);
  unsigned char* xw = smem + (size_t)wave * wlds;
  unsigned char* cw = xw + (size_t)RB * rows;  // [16][GW + 1] entries of CW bytes
  f32x4* red = reinterpret_cast<f32x4*>(smem + (size_t)WAVES * wlds);  // [WAVES][64]

  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)scales, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)biases, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);

  // 1. Small loads first: this wave's scale / bias quads; then the
  //    activation items and the weights (2).
  const int cr = lane >> 2;
  const uint32_t coff = ((uint32_t)(n0 + cr) * (uint32_t)G + (uint32_t)(u0 * GPS + 4 * (lane & 3))) * 2u;
  u32x2 sv[kLeanQuads], bv[kLeanQuads];
#pragma unroll
  for (int t = 0; t < kLeanQuads; ++t) {
    sv[t] = bv[t] = u32x2{0u, 0u};
    if (4 * t < quads) {
      sv[t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, coff + 32u * t, 0, 0));
      bv[t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(br, coff + 32u * t, 0, 0));
    }
  }
  // 2. Activations and weights.  8-bit weights with all steps in flight
  //    (IL): step j's activation items (item q: rows 4q + lane / 16, the
  //    step's 16-byte slot lane % 16) and then its weights, step by step, so
  //    the first weight steps are requested after a quarter of the
  //    activation loads instead of after all of them, and the stream waits
  //    for each step's data as it reaches the step (loads complete in
  //    order); a step's items are staged right before its operands are read
  //    (M = 4 / 16 at N = K = 4096: 6.2 -> 5.8 / 8.05 -> 7.7 us; the same
  //    order made 4-bit weights, half the bytes per step, slower: 6.1 ->
  //    6.8 us at M = 16).  Otherwise every activation item (row rr, item t:
  //    bytes 1024 t + 16 lane of the row's range), then the first PF weight
  //    steps, then the staging.
  constexpr bool IL = ONE && BITS == 8;
  const uint32_t voff = (uint32_t)(n0 + r) * rowbytes + (uint32_t)(4 * u0 + g) * CB;
  uint32_t buf[PF][BITS];
  u32x4 xv[XMAX];
  constexpr int QR = XMAX / NST;  // IL: items per step (rows <= 4 QR)
  if constexpr (IL) {
    const uint32_t xlo =
        (uint32_t)(lane >> 4) * (uint32_t)k * 2u + (uint32_t)u0 * 256u + (uint32_t)(lane & 15) * 16u;
#pragma unroll
    for (int j = 0; j < NST; ++j) {
#pragma unroll
      for (int q = 0; q < QR; ++q)
        if (4 * q < rows)
          xv[j * QR + q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         xr, xlo + 256u * j, (int)((uint32_t)(4 * q) * (uint32_t)k * 2u), 0));
      lean_load<BITS>(wr, voff + j * 4 * CB, 0, buf[j]);
    }
  } else {
    const uint32_t xoff = (uint32_t)u0 * 256u + (uint32_t)lane * 16u;
#pragma unroll
    for (int i = 0; i < XMAX; ++i) {
      const int rr = i / IPR, t = i % IPR;
      if (rr < rows)
        xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              xr, xoff + 1024u * t, (int)((uint32_t)rr * (uint32_t)k * 2u), 0));
    }
#pragma unroll
    for (int p = 0; p < PF; ++p) lean_load_nt<BITS, BITS == 4>(wr, voff + p * 4 * CB, 0, buf[p]);
#pragma unroll
    for (int i = 0; i < XMAX; ++i) {
      const int rr = i / IPR, t = i % IPR;
      if (rr < rows)
        *reinterpret_cast<u32x4*>(xw + rr * RB + 1024 * t + (lane >> 4) * 256 + (((lane & 15) ^ swz_key(rr)) << 4)) =
            interleave_x<BITS>(xv[i]);
    }
  }

  // 3. Stage this wave's constants, vote within the wave.
  FastQuick fq;
  fast_quick_init(fq);
  const int cwp = GW + 1;
#pragma unroll
  for (int t = 0; t < kLeanQuads; ++t) {
    const int cq = (lane & 3) + 4 * t;
    if (4 * t < quads && cq < quads) {
      unsigned char* dst = cw + (size_t)(cr * cwp + cq * 4) * CW;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (CW == 16) {
          reinterpret_cast<f32x4*>(dst)[2 * h] = group_consts<TT>(sv[t][h] & 0xffffu, bv[t][h] & 0xffffu);
          reinterpret_cast<f32x4*>(dst)[2 * h + 1] = group_consts<TT>(sv[t][h] >> 16, bv[t][h] >> 16);
        } else {
          reinterpret_cast<f32x2*>(dst)[2 * h] =
              f32x2{TT::to_f32((uint16_t)(sv[t][h] & 0xffffu)), TT::to_f32((uint16_t)(bv[t][h] & 0xffffu))};
          reinterpret_cast<f32x2*>(dst)[2 * h + 1] =
              f32x2{TT::to_f32((uint16_t)(sv[t][h] >> 16)), TT::to_f32((uint16_t)(bv[t][h] >> 16))};
        }
        fast_quick_add<TT>(fq, sv[t][h], bv[t][h]);
      }
    }
  }
  bool ok = true;
  if (!fast_quick_ok<TT>(fq)) {
#pragma unroll
    for (int t = 0; t < kLeanQuads; ++t) {
      const int cq = (lane & 3) + 4 * t;
      if (4 * t < quads && cq < quads) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          ok &= fast_ok_bits<TT>(sv[t][h] & 0xffffu, bv[t][h] & 0xffffu) &
                fast_ok_bits<TT>(sv[t][h] >> 16, bv[t][h] >> 16);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool fast = __builtin_amdgcn_ballot_w64(!ok) == 0;

  // 4. Stream: lane (row r, group g) reads slice i of step j at
  //    xw + r * RB + j * 256 + ((4g + i) ^ swz_key(r)) * 16.
  const unsigned char* cbase = cw + (size_t)(r * cwp + ((g * 32) >> GS_SHIFT)) * CW;
  const unsigned char* xbase = xw + r * RB;
  int xsw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xsw[i] = ((4 * g + i) ^ swz_key(r)) << 4;
  // IL: step j's activation items into its slots of rows 4q + lane / 16.
  auto stage = [&](int j) {
    if constexpr (IL) {
#pragma unroll
      for (int q = 0; q < QR; ++q) {
        const int rr = 4 * q + (lane >> 4);
        if (4 * q < rows && rr < rows)
          *reinterpret_cast<u32x4*>(xw + rr * RB + 256 * j + (((lane & 15) ^ swz_key(rr)) << 4)) =
              interleave_x<BITS>(xv[j * QR + q]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  };
  const f32x4 acc =
      fast ? lean_stream<TT, BITS, GS_SHIFT, PF, ONE, true, 16, CW>(wr, voff, nsteps, cbase, xbase, buf, xsw, stage)
           : lean_stream<TT, BITS, GS_SHIFT, PF, ONE, false, 16, CW>(wr, voff, nsteps, cbase, xbase, buf, xsw, stage);

  // 5. The waves' K ranges in order; element i of lane (r, g) is output row
  //    4g + i, column n0 + r.
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0 && n0 + r < n) {
    f32x4 v = red[lane];
#pragma unroll
    for (int i = 1; i < WAVES; ++i) v = v + red[i * 64 + lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * g + i;
      if (row < m) y[(size_t)row * n + n0 + r] = TT::from_f32(v[i]);
    }
  }
}

int shift_of(int gs) {
  int s = 0;
  while ((1 << s) < gs) ++s;
  return s;
}

template <typename TT, int BITS, int WAVES, int PF, bool EXACT>
hipError_t launch_cfg(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k,
                      size_t lds) {
  if (lds > 64 * 1024) {
    // Long rows need more than the default 64 KiB of dynamic LDS (gfx950 has
    // 160 KiB per workgroup, shared with the kernel's static LDS); raise the
    // kernel's limit once.
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&qmv_kernel<TT, BITS, WAVES, PF, EXACT>);
      hipFuncAttributes fa;
      hipError_t e = hipFuncGetAttributes(&fa, fn);
      if (e != hipSuccess) return e;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (attr != hipSuccess) return attr;
    if (lds > 160 * 1024 - 1024) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((qmv_kernel<TT, BITS, WAVES, PF, EXACT>), dim3((unsigned)((n + 15) / 16)),
                     dim3(64 * WAVES), lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), n, k, shift_of(q.gs));
  return hipGetLastError();
}

// EXACT geometry: every wave owns the same whole number of PF-step batches.
template <typename TT, int BITS, int WAVES, int PF>
hipError_t launch_pf(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k,
                     size_t lds) {
  const int chunks = k / 32;
  const bool exact = chunks % 4 == 0 && (chunks / 4) % (WAVES * PF) == 0;
  if (exact) return launch_cfg<TT, BITS, WAVES, PF, true>(s, q, x, y, n, k, lds);
  return launch_cfg<TT, BITS, WAVES, PF, false>(s, q, x, y, n, k, lds);
}

template <typename TT, int BITS, int GS_SHIFT, int WAVES, int PF, bool ONE, bool BATCH = false>
hipError_t launch_lean_cfg(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k,
                           size_t lds, int count, const BatchArgs& ba) {
  if (lds > 64 * 1024) {
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&qmv_lean_kernel<TT, BITS, GS_SHIFT, WAVES, PF, ONE, BATCH>);
      hipFuncAttributes fa;
      hipError_t e = hipFuncGetAttributes(&fa, fn);
      if (e != hipSuccess) return e;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (attr != hipSuccess) return attr;
  }
  hipLaunchKernelGGL((qmv_lean_kernel<TT, BITS, GS_SHIFT, WAVES, PF, ONE, BATCH>),
                     dim3((unsigned)((n + 15) / 16), (unsigned)count), dim3(64 * WAVES), lds, s, q.w,
                     static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                     static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), n, k, ba);
  return hipGetLastError();
}

template <typename TT, int BITS, int GS_SHIFT, int WAVES, bool BATCH = false>
hipError_t launch_lean_gs(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k,
                          size_t lds, int count = 1, const BatchArgs& ba = BatchArgs{}) {
  const int nsteps = k / (128 * WAVES);
  if (nsteps == 8) return launch_lean_cfg<TT, BITS, GS_SHIFT, WAVES, 8, true, BATCH>(s, q, x, y, n, k, lds, count, ba);
  if (nsteps == 4) return launch_lean_cfg<TT, BITS, GS_SHIFT, WAVES, 4, true, BATCH>(s, q, x, y, n, k, lds, count, ba);
  if (nsteps % 8 == 0)
    return launch_lean_cfg<TT, BITS, GS_SHIFT, WAVES, 8, false, BATCH>(s, q, x, y, n, k, lds, count, ba);
  return launch_lean_cfg<TT, BITS, GS_SHIFT, WAVES, 4, false, BATCH>(s, q, x, y, n, k, lds, count, ba);
}

template <typename TT, int BITS, int WAVES, bool BATCH = false>
hipError_t launch_lean_w(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k,
                         size_t lds, int count = 1, const BatchArgs& ba = BatchArgs{}) {
  if (q.gs == 32) return launch_lean_gs<TT, BITS, 5, WAVES, BATCH>(s, q, x, y, n, k, lds, count, ba);
  if (q.gs == 64) return launch_lean_gs<TT, BITS, 6, WAVES, BATCH>(s, q, x, y, n, k, lds, count, ba);
  return launch_lean_gs<TT, BITS, 7, WAVES, BATCH>(s, q, x, y, n, k, lds, count, ba);
}

// The lean kernel's shape contract: K a multiple of 512 * waves (each wave a
// whole number of 4-step batches), at most 16384 activations and 128 groups
// per row in one wave's K range, 32-bit buffer ranges, 8-byte aligned scales
// and biases.
template <int BITS>
bool lean_fits(const QuantArgs& q, int n, int k, int waves) {
  if (BITS != 4 && BITS != 8) return false;
  if (q.gs != 32 && q.gs != 64 && q.gs != 128) return false;
  if (k % (512 * waves) != 0 || k > 16384 || (k / waves) / q.gs > 4 * kLeanQuads * 4) return false;
  if ((uint64_t)n * (uint64_t)k * BITS / 8 >= (1ull << 31)) return false;
  if ((uint64_t)n * (uint64_t)(k / q.gs) * 2 >= (1ull << 31)) return false;
  return ((reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases)) & 7u) == 0;
}

template <typename TT, int BITS, int GS_SHIFT, int NST, bool BATCH, int CW, int WAVES = 8>
hipError_t launch_rows_cfg(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                           size_t lds, int count, const BatchArgs& ba) {
  if (lds > 64 * 1024) {
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&qmm_lean_rows_kernel<TT, BITS, GS_SHIFT, WAVES, NST, BATCH, CW>);
      hipFuncAttributes fa;
      hipError_t e = hipFuncGetAttributes(&fa, fn);
      if (e != hipSuccess) return e;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (attr != hipSuccess) return attr;
  }
  hipLaunchKernelGGL((qmm_lean_rows_kernel<TT, BITS, GS_SHIFT, WAVES, NST, BATCH, CW>),
                     dim3((unsigned)((n + 15) / 16), (unsigned)count), dim3(64 * WAVES), lds, s, q.w,
                     static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                     static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), m, n, k, ba);
  return hipGetLastError();
}

constexpr size_t kRowsLdsMax = 160 * 1024 - 1024;

size_t rows_lds(int m, int k, int gs, int cw = 16) {
  const int nst = k / 1024;
  return (size_t)8 * lean_wave_lds(nst, shift_of(gs), std::min(m, 16), cw) + (size_t)8 * 64 * 16;
}

// Bytes per group's constants: 16 where they fit, else 8 at gs 32 (16 rows
// at K = 4096: 170 KiB with 16, 156.5 KiB with 8).
int rows_cw(int m, int k, int gs) { return rows_lds(m, k, gs) <= kRowsLdsMax || gs != 32 ? 16 : 8; }

template <typename TT, int BITS, int GS_SHIFT, bool BATCH, int CW>
hipError_t launch_rows_nst(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                           size_t lds, int count, const BatchArgs& ba) {
  const int nst = k / 1024;
  if (nst == 4) return launch_rows_cfg<TT, BITS, GS_SHIFT, 4, BATCH, CW>(s, q, x, y, m, n, k, lds, count, ba);
  if (nst == 8) return launch_rows_cfg<TT, BITS, GS_SHIFT, 8, BATCH, CW>(s, q, x, y, m, n, k, lds, count, ba);
  return launch_rows_cfg<TT, BITS, GS_SHIFT, 16, BATCH, CW>(s, q, x, y, m, n, k, lds, count, ba);
}

template <typename TT, int BITS, int GS_SHIFT, bool BATCH>
hipError_t launch_rows_gs(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                          int count, const BatchArgs& ba) {
  // 8-bit rows at K = 4096 and up to 8 of them: 4 waves of 8 steps (two
  // items per row and lane) instead of 8 waves of 4 (8-bit M = 8: 8.02 ->
  // 6.91 us, M = 2: 6.43 -> 5.93 us at N = 4096); 4-bit measured 5-8 %
  // faster with 8 waves.  CPQ_ROWS_WAVES = 4 or 8 forces the choice (tuning
  // hook, read once per process).
  static const int forced_w = env_int("CPQ_ROWS_WAVES", 0);
  const bool four = forced_w == 4 || (forced_w != 8 && BITS == 8);
  if (four && k == 4096 && m <= 8) {
    const size_t lds4 = (size_t)4 * lean_wave_lds(8, GS_SHIFT, std::min(m, 16)) + (size_t)4 * 64 * 16;
    return launch_rows_cfg<TT, BITS, GS_SHIFT, 8, BATCH, 16, 4>(s, q, x, y, m, n, k, lds4, count, ba);
  }
  if constexpr (GS_SHIFT == 5) {
    if (rows_cw(m, k, q.gs) == 8)
      return launch_rows_nst<TT, BITS, GS_SHIFT, BATCH, 8>(s, q, x, y, m, n, k, rows_lds(m, k, q.gs, 8), count, ba);
  }
  return launch_rows_nst<TT, BITS, GS_SHIFT, BATCH, 16>(s, q, x, y, m, n, k, rows_lds(m, k, q.gs), count, ba);
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k) {
  const size_t G = (size_t)k / q.gs;
  const size_t lds = (size_t)k * 2 + 16 * (G + 1) * 16 + 8 * 16 * 4;
  if constexpr (BITS == 4 || BITS == 8) {
    // Few row blocks (under two per CU) and K past 4096: 8 waves per block
    // keep two waves per SIMD; 12 (three per SIMD) where K splits into 12
    // ranges of at least 8 steps (K = 12288: 9.2 -> 8.4 us at N = 4096).  Up
    // to K = 4096 a 4-wave block has every step of its range in flight at
    // once, and splitting K further only adds per-wave work (8-bit, N = 4096:
    // 6.82 -> 5.93 us; 4-bit within 2 %).
    static const int forced = env_int("CPQ_QMV_WAVES", 0);  // tuning hook: 4, 8 or 12
    const bool few = (n + 15) / 16 < 512 && k > 4096;
    const int waves = forced == 4 || forced == 8 || forced == 12 ? (lean_fits<BITS>(q, n, k, forced) ? forced : 4)
                      : few && lean_fits<BITS>(q, n, k, 12) && k / (128 * 12) >= 8 ? 12
                      : few && lean_fits<BITS>(q, n, k, 8)                          ? 8
                                                                                    : 4;
    if (lean_fits<BITS>(q, n, k, waves)) {
      const int sh = shift_of(q.gs);
      const size_t llds = (size_t)waves * lean_wave_lds(k / (128 * waves), sh) + (size_t)waves * 16 * 4;
      if (llds <= 160 * 1024 - 1024) {
        if (waves == 12) return launch_lean_w<TT, BITS, 12>(s, q, x, y, n, k, llds);
        if (waves == 8) return launch_lean_w<TT, BITS, 8>(s, q, x, y, n, k, llds);
        return launch_lean_w<TT, BITS, 4>(s, q, x, y, n, k, llds);
      }
    }
  }
  if constexpr (BITS == 4 || BITS == 8) {
    // Rows of up to 1024 elements (the lean kernel takes none of them; the
    // reference's K = 896 projections and their K-padded twins): the
    // routed-decode kernel's dense form with one row, K split so that a
    // zero-padded K (896 -> 960 -> 1024) gives the same bits (lm_head,
    // N = 151936: 32.8 -> 20 us).  CPQ_QMV_DENSE=0 keeps it off (tuning
    // hook).
    const bool al16 = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q.w)) & 15u) == 0;
    if (k <= 1024 && al16 && env_int("CPQ_QMV_DENSE", 1) != 0 && dense_small_supported(q, 1, n, k))
      return launch_dense_small(s, q, x, y, 1, n, k, true);
  }
  if (lds > 160 * 1024) {
    // Very long rows: the small-M kernel while its slab constants fit in LDS
    // (about 500 groups per row), beyond that a prefill kernel, which keeps
    // no per-row constants in LDS.
    if (skinny_fits(k, q.gs)) return launch_qmm_skinny(s, q, x, y, 1, n, k);
    return launch_qmm_unsplit(s, q, x, y, 1, n, k);
  }
  const int units = k / 128;
  if constexpr (BITS == 4) {
    // Few row blocks: split K over more waves to keep enough loads in flight.
    if ((n + 15) / 16 >= 512) {
      if (units % 32 == 0) return launch_pf<TT, BITS, 4, 8>(s, q, x, y, n, k, lds);
      return launch_pf<TT, BITS, 4, 4>(s, q, x, y, n, k, lds);
    }
    if (units % 64 == 0) return launch_pf<TT, BITS, 8, 8>(s, q, x, y, n, k, lds);
    return launch_pf<TT, BITS, 8, 4>(s, q, x, y, n, k, lds);
  } else if constexpr (BITS == 8) {
    if ((n + 15) / 16 >= 512) return launch_pf<TT, BITS, 4, 4>(s, q, x, y, n, k, lds);
    return launch_pf<TT, BITS, 8, 4>(s, q, x, y, n, k, lds);
  } else {
    return launch_cfg<TT, BITS, 4, 4, false>(s, q, x, y, n, k, lds);
  }
}

template <typename TT>
hipError_t launch_bits(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k) {
  switch (q.bits) {
    case 2: return launch_t<TT, 2>(s, q, x, y, n, k);
    case 3: return launch_t<TT, 3>(s, q, x, y, n, k);
    case 4: return launch_t<TT, 4>(s, q, x, y, n, k);
    case 5: return launch_t<TT, 5>(s, q, x, y, n, k);
    case 6: return launch_t<TT, 6>(s, q, x, y, n, k);
    case 8: return launch_t<TT, 8>(s, q, x, y, n, k);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// Up to 16 rows on the lean layout: 4/8-bit, gs 32/64/128, K in
// {4096, 8192, 16384} (8 waves of 4, 8 or 16 steps), M * K / 1024 <= 64
// activation items per lane, LDS within the CU, 32-bit buffer ranges,
// 8-byte aligned scales and biases, 16-byte aligned x.
bool qmv_rows_fits(const QuantArgs& q, int m, int n, int k, const void* x) {
  if ((q.bits != 4 && q.bits != 8) || (q.dtype != CPQ_DTYPE_BF16 && q.dtype != CPQ_DTYPE_F16)) return false;
  if (q.gs != 32 && q.gs != 64 && q.gs != 128) return false;
  if (m < 1 || m > 16 || n < 1 || (k != 4096 && k != 8192 && k != 16384)) return false;
  if (m * (k / 1024) > 64) return false;
  if (rows_lds(m, k, q.gs, rows_cw(m, k, q.gs)) > kRowsLdsMax) return false;
  if ((uint64_t)n * (uint64_t)k * q.bits / 8 >= (1ull << 31)) return false;
  if ((uint64_t)n * (uint64_t)(k / q.gs) * 2 >= (1ull << 31)) return false;
  if ((uint64_t)m * (uint64_t)k * 2 >= (1ull << 31)) return false;
  return ((reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases)) & 7u) == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

template <bool BATCH>
hipError_t launch_rows_any(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int count,
                           const BatchArgs& ba) {
  auto by_gs = [&](auto tt, auto bits) -> hipError_t {
    using TT = decltype(tt);
    constexpr int B = decltype(bits)::value;
    if (q.gs == 32) return launch_rows_gs<TT, B, 5, BATCH>(s, q, x, y, m, n, k, count, ba);
    if (q.gs == 64) return launch_rows_gs<TT, B, 6, BATCH>(s, q, x, y, m, n, k, count, ba);
    return launch_rows_gs<TT, B, 7, BATCH>(s, q, x, y, m, n, k, count, ba);
  };
  using B4 = std::integral_constant<int, 4>;
  using B8 = std::integral_constant<int, 8>;
  if (q.dtype == CPQ_DTYPE_BF16) return q.bits == 4 ? by_gs(BF16{}, B4{}) : by_gs(BF16{}, B8{});
  if (q.dtype == CPQ_DTYPE_F16) return q.bits == 4 ? by_gs(F16{}, B4{}) : by_gs(F16{}, B8{});
  return hipErrorInvalidValue;
}

hipError_t launch_qmv_rows(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  return launch_rows_any<false>(s, q, x, y, m, n, k, 1, BatchArgs{});
}

hipError_t launch_qmv_rows_batched(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                                   int count, const BatchArgs& ba) {
  if (count < 1 || count > 65535) return hipErrorInvalidValue;
  return launch_rows_any<true>(s, q, x, y, m, n, k, count, ba);
}

// The batched decode kernel runs 4 waves per workgroup (the batch fills the
// grid): the lean kernel's contract at 4 waves, LDS within the CU.
bool qmv_batch_fits(const QuantArgs& q, int n, int k) {
  if (q.dtype != CPQ_DTYPE_BF16 && q.dtype != CPQ_DTYPE_F16) return false;
  const bool fits = q.bits == 4 ? lean_fits<4>(q, n, k, 4) : q.bits == 8 ? lean_fits<8>(q, n, k, 4) : false;
  if (!fits) return false;
  return (size_t)4 * lean_wave_lds(k / 512, shift_of(q.gs)) + (size_t)4 * 16 * 4 <= 160 * 1024 - 1024;
}

hipError_t launch_qmv_batched(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k, int count,
                              const BatchArgs& ba) {
  if (count < 1 || count > 65535 || !qmv_batch_fits(q, n, k)) return hipErrorInvalidValue;
  const size_t lds = (size_t)4 * lean_wave_lds(k / 512, shift_of(q.gs)) + (size_t)4 * 16 * 4;
  if (q.dtype == CPQ_DTYPE_BF16)
    return q.bits == 4 ? launch_lean_w<BF16, 4, 4, true>(s, q, x, y, n, k, lds, count, ba)
                       : launch_lean_w<BF16, 8, 4, true>(s, q, x, y, n, k, lds, count, ba);
  return q.bits == 4 ? launch_lean_w<F16, 4, 4, true>(s, q, x, y, n, k, lds, count, ba)
                     : launch_lean_w<F16, 8, 4, true>(s, q, x, y, n, k, lds, count, ba);
}

hipError_t launch_qmv(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k) {
  if (q.dtype == CPQ_DTYPE_BF16) return launch_bits<BF16>(s, q, x, y, n, k);
  if (q.dtype == CPQ_DTYPE_F16) return launch_bits<F16>(s, q, x, y, n, k);
  return hipErrorInvalidValue;
}

}  // namespace cpq
