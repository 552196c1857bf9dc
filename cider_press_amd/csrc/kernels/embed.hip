// embed_tokens for gfx950: out[t, :] = RNE_T(fmaf(scale, q, bias)) over row
// ids[t] of a quantized [vocab, hidden] table.
//
// Reference: crates/cider-press-models/src/nn.rs:123-136 (embed_tokens) runs
// three Tensor::gather dispatches (packed words, scales, biases;
// runtime/src/tensor.rs:1444-1530) and one affine_dequantize over the
// gathered triple (quantized.h:2543-2603).  Here the gather is folded into
// the dequantization: each thread reads a 32-element chunk of the selected
// row straight from the table and writes its T values, so the gathered
// triple is never materialised.  Arithmetic is the dequantize kernel's, so
// the output is bit-identical to gather-then-dequantize.
//
// HBM-bound: algorithmic bytes per token = hidden*bits/8 (row words)
// + 2*(hidden/gs)*sizeof(T) (scales, biases) + hidden*sizeof(T) (output)
// + 4 (id).  Ids at or past `vocab` give a zero row and are counted in the
// session's status word, which the next wait reports.
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

template <typename TT, int BITS>
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* __restrict__ w,
                                                    const uint16_t* __restrict__ scales,
                                                    const uint16_t* __restrict__ biases,
                                                    const uint32_t* __restrict__ ids, uint32_t n_chunks,
                                                    uint32_t row_chunks, uint32_t vocab, int gs_shift,
                                                    uint16_t* __restrict__ out, unsigned int* bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t c = blockIdx.x * blockDim.x + threadIdx.x; c < n_chunks; c += stride) {
    const uint32_t t = c / row_chunks, j = c - t * row_chunks;
    const uint32_t id = ids[t];
    u32x4* dst = reinterpret_cast<u32x4*>(out + (size_t)c * 32);
    if (id >= vocab) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = u32x4{0u, 0u, 0u, 0u};
      if (j == 0) atomicAdd(bad, 1u);
      continue;
    }
    const size_t src = (size_t)id * row_chunks + j;  // chunk index in the table
    uint32_t wv[BITS];
    load_chunk<BITS>(w, src, wv);
    const size_t g = (src * 32) >> gs_shift;
    const float s = TT::to_f32(scales[g]);
    const float b = TT::to_f32(biases[g]);
    uint32_t o[16];
    dequant_chunk<TT, BITS>(wv, s, b, o);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
  }
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const uint32_t* ids, uint32_t n_ids, uint32_t vocab,
                    uint32_t hidden, void* out, unsigned int* bad) {
  const uint32_t row_chunks = hidden / 32;
  const uint32_t n_chunks = n_ids * row_chunks;  // the caller bounds this below 2^31
  if (n_chunks == 0) return hipSuccess;
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  uint32_t blocks = (n_chunks + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  hipLaunchKernelGGL((embed_kernel<TT, BITS>), dim3(blocks), dim3(256), 0, s, q.w,
                     static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases), ids,
                     n_chunks, row_chunks, vocab, gs_shift, static_cast<uint16_t*>(out), bad);
  return hipGetLastError();
}

template <typename TT>
hipError_t launch_bits(hipStream_t s, const QuantArgs& q, const uint32_t* ids, uint32_t n_ids, uint32_t vocab,
                       uint32_t hidden, void* out, unsigned int* bad) {
  switch (q.bits) {
    case 2: return launch_t<TT, 2>(s, q, ids, n_ids, vocab, hidden, out, bad);
    case 3: return launch_t<TT, 3>(s, q, ids, n_ids, vocab, hidden, out, bad);
    case 4: return launch_t<TT, 4>(s, q, ids, n_ids, vocab, hidden, out, bad);
    case 5: return launch_t<TT, 5>(s, q, ids, n_ids, vocab, hidden, out, bad);
    case 6: return launch_t<TT, 6>(s, q, ids, n_ids, vocab, hidden, out, bad);
    case 8: return launch_t<TT, 8>(s, q, ids, n_ids, vocab, hidden, out, bad);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_embed(hipStream_t s, const QuantArgs& q, const uint32_t* ids, uint32_t n_ids, uint32_t vocab,
                        uint32_t hidden, void* out, unsigned int* bad) {
  if (q.dtype == CPQ_DTYPE_BF16) return launch_bits<BF16>(s, q, ids, n_ids, vocab, hidden, out, bad);
  if (q.dtype == CPQ_DTYPE_F16) return launch_bits<F16>(s, q, ids, n_ids, vocab, hidden, out, bad);
  return hipErrorInvalidValue;
}

}  // namespace cpq
