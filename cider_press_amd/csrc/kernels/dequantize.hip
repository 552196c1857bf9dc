// affine_dequantize for gfx950: out[i] = RNE_T(fmaf(scale, q_i, bias)).
//
// Reference semantics: kernels-mlx/mlx/backend/metal/kernels/quantized.h:2543-2603
// (one thread per packed byte there).  4- and 8-bit: a wave takes 256
// consecutive 8-element pieces (one word at 4-bit, two at 8-bit) per
// iteration, lane l the pieces l, l + 64, l + 128, l + 192, so each load
// instruction reads 256 (512) contiguous bytes and each 16-byte store
// instruction writes 1 KiB contiguous.  Other widths (elements straddle
// words): one thread per 32-element chunk (`bits` words in, 64 bytes out).
// Algorithmic bytes per element: bits/8 (weights) + 2*sizeof(T)/gs
// (scale, bias) + sizeof(T) (output).
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

template <typename TT, int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         uint16_t* __restrict__ out,
                                                         size_t n_chunks, int gs_shift) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < n_chunks; c += stride) {
    uint32_t wv[BITS];
    load_chunk<BITS>(w, c, wv);
    const size_t g = (c * 32) >> gs_shift;
    const float s = TT::to_f32(scales[g]);
    const float b = TT::to_f32(biases[g]);
    uint32_t o[16];
    dequant_chunk<TT, BITS>(wv, s, b, o);
    u32x4* dst = reinterpret_cast<u32x4*>(out + c * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = {o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
      dst[i] = v;
    }
  }
}

// 8-element piece p: words BITS/4 words from word p * BITS / 4.
template <int BITS>
__device__ __forceinline__ void load_piece(const uint32_t* __restrict__ w, size_t p, uint32_t* wv) {
  if constexpr (BITS == 4) {
    wv[0] = w[p];
  } else {
    const u32x2 v = *reinterpret_cast<const u32x2*>(w + 2 * p);
    wv[0] = v.x;
    wv[1] = v.y;
  }
}

template <typename TT, int BITS>
__global__ __launch_bounds__(256) void dequantize_pieces_kernel(const uint32_t* __restrict__ w,
                                                                const uint16_t* __restrict__ scales,
                                                                const uint16_t* __restrict__ biases,
                                                                uint16_t* __restrict__ out, size_t n_pieces,
                                                                int gs_shift) {
  static_assert(BITS == 4 || BITS == 8, "whole words per piece");
  const int lane = threadIdx.x & 63;
  const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const size_t waves = ((size_t)gridDim.x * blockDim.x) >> 6;
  for (size_t base = wave * 256; base < n_pieces; base += waves * 256) {
    uint32_t wv[4][BITS / 4];
    uint16_t sv[4], bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const size_t p = base + lane + 64 * j;
      if (p < n_pieces) {
        load_piece<BITS>(w, p, wv[j]);
        const size_t g = (p * 8) >> gs_shift;
        sv[j] = scales[g];
        bv[j] = biases[g];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const size_t p = base + lane + 64 * j;
      if (p < n_pieces) {
        const float sc = TT::to_f32(sv[j]), b = TT::to_f32(bv[j]);
        uint32_t o[4];
        dequant8<TT, BITS, 0>(wv[j], sc, sc * 0.0625f, b, o);
        *reinterpret_cast<u32x4*>(out + p * 8) = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, void* out, size_t n_out) {
  const size_t n_chunks = n_out / 32;
  if (n_chunks == 0) return hipSuccess;
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  const int block = 256;
  if constexpr (BITS == 4 || BITS == 8) {
    const size_t n_pieces = n_out / 8;
    size_t pblocks = (n_pieces + 1023) / 1024;  // 4 waves x 256 pieces per block and iteration
    if (pblocks > 256 * 16) pblocks = 256 * 16;
    hipLaunchKernelGGL((dequantize_pieces_kernel<TT, BITS>), dim3((unsigned)pblocks), dim3(block), 0, s, q.w,
                       static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                       static_cast<uint16_t*>(out), n_pieces, gs_shift);
    return hipGetLastError();
  }
  size_t blocks = (n_chunks + block - 1) / block;
  // Grid-stride beyond ~64 waves per CU buys nothing.
  if (blocks > 256 * 64) blocks = 256 * 64;
  hipLaunchKernelGGL((dequantize_kernel<TT, BITS>), dim3((unsigned)blocks), dim3(block), 0, s,
                     q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<uint16_t*>(out),
                     n_chunks, gs_shift);
  return hipGetLastError();
}

template <typename TT>
hipError_t launch_bits(hipStream_t s, const QuantArgs& q, void* out, size_t n_out) {
  switch (q.bits) {
    case 2: return launch_t<TT, 2>(s, q, out, n_out);
    case 3: return launch_t<TT, 3>(s, q, out, n_out);
    case 4: return launch_t<TT, 4>(s, q, out, n_out);
    case 5: return launch_t<TT, 5>(s, q, out, n_out);
    case 6: return launch_t<TT, 6>(s, q, out, n_out);
    case 8: return launch_t<TT, 8>(s, q, out, n_out);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_dequantize(hipStream_t s, const QuantArgs& q, void* out, size_t n_out) {
  if (q.dtype == CPQ_DTYPE_BF16) return launch_bits<BF16>(s, q, out, n_out);
  if (q.dtype == CPQ_DTYPE_F16) return launch_bits<F16>(s, q, out, n_out);
  return hipErrorInvalidValue;
}

}  // namespace cpq
