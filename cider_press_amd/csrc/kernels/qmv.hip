// Decode GEMV (M = 1) for gfx950: y[n] = sum_k x[k] * RNE_T(fmaf(s, q[n,k], b)).
//
// Reference op: affine_qmv_fast / affine_qmv (kernels-mlx/.../quantized.h:749-975),
// dispatched by crates/cider-press-kernels/src/kernels/qmv.rs:77-205.
// Numerics follow the dequantize-then-dot contract (weights rounded to T,
// fp32 accumulation) rather than MLX's unrounded factored form: with bf16
// outputs the factored form exceeds the 2e-3 relative-L2 budget at K=4096.
//
// HBM-bound: algorithmic bytes per call = N*K*bits/8 + 2*N*(K/gs)*sizeof(T)
// + (K + N)*sizeof(T).  The whole cost per weight is VALU dequantization, so
// the dot products go to the matrix cores:
//   - a workgroup owns 16 output rows and splits K over its WAVES waves;
//   - the activation row is staged once into LDS, permuted into the
//     interleaved slot order of the dequantizer (common.hpp), together with
//     the 16 rows' (scale, bias) pairs and a workgroup-wide check that the
//     single-FMA fast dequantization is exact for every group;
//   - lane l streams row n0 + l%16, chunk 4u + l/16 (16 B of packed 4-bit
//     weights: the 4 lane groups of a wave read 64 contiguous bytes of each
//     of 16 rows), keeping PF chunks in flight per lane;
//   - each 8-element slice is dequantized into an MFMA B operand and issued
//     as v_mfma_f32_16x16x32 against the activation slice broadcast to all 16
//     A rows (the matrix cores are otherwise idle at M = 1);
//   - the K-partial results of the waves are summed through LDS.
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

template <int BITS>
struct QmvPrefetch {
  static constexpr int PF = BITS <= 4 ? 8 : 4;  // chunks in flight per lane
};

template <typename TT, int BITS, int WAVES, bool FAST>
__device__ __forceinline__ f32x4 qmv_stream(const uint32_t* __restrict__ wrow, bool row_ok,
                                            const uint16_t* xs, const uint32_t* sbrow, int chunks,
                                            int gs_shift, int wave, int g) {
  constexpr int PF = QmvPrefetch<BITS>::PF;
  const int units = (chunks + 3) >> 2;
  const int nsteps = units > wave ? (units - wave + WAVES - 1) / WAVES : 0;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  uint32_t buf[PF][BITS];

  auto chunk_of = [&](int j) { return 4 * (wave + WAVES * j) + g; };
  auto fetch = [&](int j, uint32_t* dst) {
    const int c = chunk_of(j);
    if (row_ok && c < chunks) {
      load_chunk<BITS>(wrow, (size_t)c, dst);
    } else {
#pragma unroll
      for (int i = 0; i < BITS; ++i) dst[i] = 0u;
    }
  };

#pragma unroll
  for (int p = 0; p < PF; ++p)
    if (p < nsteps) fetch(p, buf[p]);

  for (int base = 0; base < nsteps; base += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int j = base + p;
      if (j < nsteps) {
        uint32_t cur[BITS];
#pragma unroll
        for (int i = 0; i < BITS; ++i) cur[i] = buf[p][i];
        if (j + PF < nsteps) fetch(j + PF, buf[p]);
        const int c = chunk_of(j);
        const bool live = c < chunks;
        const uint32_t sb = live ? sbrow[(c << 5) >> gs_shift] : 0u;
        const float s = TT::to_f32((uint16_t)(sb & 0xffffu));
        const float b = TT::to_f32((uint16_t)(sb >> 16));
        const float s16 = s * 0.0625f;
        const float c0 = FAST ? fmaf(-1024.f, s, b) : 0.f;
        const float c1 = FAST ? fmaf(-64.f, s, b) : 0.f;
        const u32x4* xa = reinterpret_cast<const u32x4*>(xs + (live ? c : 0) * 32);
        const u32x4 zero = {0u, 0u, 0u, 0u};
        acc = Mfma16<TT>::run(live ? xa[0] : zero, dequant_slice<TT, BITS, FAST, 0>(cur, s, s16, b, c0, c1), acc);
        acc = Mfma16<TT>::run(live ? xa[1] : zero, dequant_slice<TT, BITS, FAST, 1>(cur, s, s16, b, c0, c1), acc);
        acc = Mfma16<TT>::run(live ? xa[2] : zero, dequant_slice<TT, BITS, FAST, 2>(cur, s, s16, b, c0, c1), acc);
        acc = Mfma16<TT>::run(live ? xa[3] : zero, dequant_slice<TT, BITS, FAST, 3>(cur, s, s16, b, c0, c1), acc);
      }
    }
  }
  return acc;
}

template <typename TT, int BITS, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void qmv_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int n, int k,
                                                         int gs_shift) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int G = k >> gs_shift;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);                 // k elements, interleaved
  uint32_t* sb = reinterpret_cast<uint32_t*>(smem + (size_t)k * 2);  // [16][G] (scale | bias << 16)
  float* red = reinterpret_cast<float*>(smem + (size_t)k * 2 + (size_t)16 * G * 4);  // [WAVES][16]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int row = n0 + nl;
  const bool row_ok = row < n;
  const int chunks = k >> 5;
  const size_t words_per_row = (size_t)k * BITS / 32;
  const uint32_t* wrow = w + (size_t)(row_ok ? row : 0) * words_per_row;

  // Stage the activation (interleaved per 8-element slice).
  for (int i = tid; i < (k >> 3); i += 64 * WAVES) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    *reinterpret_cast<u32x4*>(xs + (size_t)i * 8) = interleave_x<BITS>(v);
  }
  // Stage (scale, bias) of the 16 rows and decide the dequantization path.
  bool ok = true;
  for (int i = tid; i < 16 * G; i += 64 * WAVES) {
    const int r = i / G, gi = i - r * G;
    const int rr = n0 + r;
    uint16_t sv = 0, bv = 0;
    if (rr < n) {
      sv = scales[(size_t)rr * G + gi];
      bv = biases[(size_t)rr * G + gi];
    }
    sb[i] = (uint32_t)sv | ((uint32_t)bv << 16);
    ok = ok && fast_ok<TT>(TT::to_f32(sv), TT::to_f32(bv));
  }
  const bool fast = __syncthreads_and(ok);

  const uint32_t* sbrow = sb + nl * G;
  f32x4 acc;
  if (fast)
    acc = qmv_stream<TT, BITS, WAVES, true>(wrow, row_ok, xs, sbrow, chunks, gs_shift, wave, g);
  else
    acc = qmv_stream<TT, BITS, WAVES, false>(wrow, row_ok, xs, sbrow, chunks, gs_shift, wave, g);

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

int shift_of(int gs) {
  int s = 0;
  while ((1 << s) < gs) ++s;
  return s;
}

template <typename TT, int BITS, int WAVES>
hipError_t launch_w(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k,
                    size_t lds) {
  hipLaunchKernelGGL((qmv_kernel<TT, BITS, WAVES>), dim3((unsigned)((n + 15) / 16)), dim3(64 * WAVES),
                     lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), n, k, shift_of(q.gs));
  return hipGetLastError();
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k) {
  const size_t G = (size_t)k / q.gs;
  const size_t lds = (size_t)k * 2 + 16 * G * 4 + 8 * 16 * 4;
  if (lds > 64 * 1024)  // very long rows: the LDS-free small-M kernel
    return launch_qmm_skinny(s, q, x, y, 1, n, k);
  // Few row blocks: split K over more waves to keep enough loads in flight.
  if ((n + 15) / 16 >= 512) return launch_w<TT, BITS, 4>(s, q, x, y, n, k, lds);
  return launch_w<TT, BITS, 8>(s, q, x, y, n, k, lds);
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

hipError_t launch_qmv(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k) {
  if (q.dtype == CPQ_DTYPE_BF16) return launch_bits<BF16>(s, q, x, y, n, k);
  if (q.dtype == CPQ_DTYPE_F16) return launch_bits<F16>(s, q, x, y, n, k);
  return hipErrorInvalidValue;
}

}  // namespace cpq
