// affine_dequantize for gfx950: out[i] = RNE_T(fmaf(scale, q_i, bias)).
//
// Reference semantics: kernels-mlx/mlx/backend/metal/kernels/quantized.h:2543-2603
// (one thread per packed byte there).  Here one thread owns a 32-element
// chunk (`bits` words in, 64 bytes of T out): a 16-byte load and four 16-byte
// stores per thread for 4-bit, so the kernel streams at HBM rate.
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

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, void* out, size_t n_out) {
  const size_t n_chunks = n_out / 32;
  if (n_chunks == 0) return hipSuccess;
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  const int block = 256;
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
