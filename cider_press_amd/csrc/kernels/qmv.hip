// Decode GEMV (M = 1) for gfx950: y[n] = sum_k x[k] * RNE_T(fmaf(s, q[n,k], b)).
//
// Reference op: affine_qmv_fast / affine_qmv (kernels-mlx/.../quantized.h:749-975),
// dispatched by crates/cider-press-kernels/src/kernels/qmv.rs:77-205.
// Numerics follow the dequantize-then-dot contract (weights rounded to T,
// fp32 accumulation) rather than MLX's unrounded factored form: with bf16
// outputs the factored form exceeds the 2e-3 relative-L2 budget at K=4096.
//
// Mapping: one wave64 owns ROWS consecutive output rows.  Lane l walks the
// row in 32-element chunks c = l, l+64, ...: one 16-byte load of packed
// 4-bit weights per row per chunk (a wave reads 1 KiB contiguous per row),
// the matching 32 activations (64 B, shared by the ROWS rows) and one
// scale/bias pair.  Weights are dequantized in registers to packed T pairs
// and reduced with v_dot2_f32_{bf16,f16}; a butterfly over the wave gives
// each row's sum.  HBM-bound: algorithmic bytes per row = K*bits/8 +
// 2*(K/gs)*sizeof(T), plus x and y once.
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

template <typename TT, int BITS, int ROWS>
__global__ __launch_bounds__(256) void qmv_kernel(const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases,
                                                  const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ y, int n, int k,
                                                  int gs_shift) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int row0 = wave * ROWS;
  if (row0 >= n) return;
  const int chunks = k >> 5;
  const size_t words_per_row = (size_t)k * BITS / 32;
  const int groups_per_row = k >> gs_shift;

  const uint32_t* wrow[ROWS];
  const uint16_t* srow[ROWS];
  const uint16_t* brow[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int row = min(row0 + r, n - 1);  // tail rows recompute the last row; stores are guarded
    wrow[r] = w + (size_t)row * words_per_row;
    srow[r] = scales + (size_t)row * groups_per_row;
    brow[r] = biases + (size_t)row * groups_per_row;
  }

  float acc0[ROWS], acc1[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) acc0[r] = acc1[r] = 0.f;

  for (int c = lane; c < chunks; c += 64) {
    uint32_t xp[16];
    const u32x4* xs = reinterpret_cast<const u32x4*>(x + (size_t)c * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = xs[i];
      xp[4 * i] = v.x; xp[4 * i + 1] = v.y; xp[4 * i + 2] = v.z; xp[4 * i + 3] = v.w;
    }
    const int g = (c << 5) >> gs_shift;
    uint32_t wv[ROWS][BITS];
    float sv[ROWS], bv[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      load_chunk<BITS>(wrow[r], (size_t)c, wv[r]);
      sv[r] = TT::to_f32(srow[r][g]);
      bv[r] = TT::to_f32(brow[r][g]);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      uint32_t wp[16];
      dequant_chunk<TT, BITS>(wv[r], sv[r], bv[r], wp);
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        acc0[r] = TT::dot2(wp[i], xp[i], acc0[r]);
        acc1[r] = TT::dot2(wp[i + 1], xp[i + 1], acc1[r]);
      }
    }
  }

#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const float v = wave_sum(acc0[r] + acc1[r]);
    if (lane == r && row0 + r < n) y[row0 + r] = TT::from_f32(v);
  }
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k) {
  constexpr int ROWS = 4;
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  const int waves = (n + ROWS - 1) / ROWS;
  const int blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((qmv_kernel<TT, BITS, ROWS>), dim3(blocks), dim3(256), 0, s, q.w,
                     static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                     static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), n, k, gs_shift);
  return hipGetLastError();
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
