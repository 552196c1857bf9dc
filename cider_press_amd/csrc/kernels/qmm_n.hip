// Non-transposed quantized matmul (MLX transpose=false) for gfx950:
//   Y[M, N] = X[M, K] . dequant(W)      with W logically [K, N]: row k holds
//   N values packed along N (N*bits/32 words) and N/gs (scale, bias) groups.
//
// Reference ops: affine_qvm / affine_qmm_n (kernels-mlx/.../quantized.h:
// 977-1086 qvm_impl, 1215-1349 qmm_n_impl; kernels :1600-1712, 1845-1903).
// The reference's runtime does not route to them (tensor.rs:2069-2075
// rejects transpose=false); they complete the MLX op surface.  Contract as
// for qmm_t: weights dequantized to T exactly as affine_dequantize does,
// fp32 accumulation, T out.
//
// The MFMA operands want 8 consecutive k per lane, while a row of W is
// contiguous along n.  Each K-step therefore dequantizes its 64 x 64 W tile
// (one 32-column chunk per thread: one (scale, bias) group, the shared
// bit-exact chunk dequantizer) and writes it transposed into LDS ([n][k]);
// the activation tile is staged as is ([m][k]).  Four waves then run
// v_mfma_f32_16x16x32 on 32 x 32 quadrants of the 64 x 64 output tile.
// qvm (M = 1) is the same kernel with one row tile.  Grids with few tiles
// split K over blockIdx.z: each part stores an fp32 partial tile, and a
// second kernel adds the parts in order (deterministic) and rounds to T.
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int NT_M = 64, NT_N = 64, NT_K = 64;
constexpr int NT_P = NT_K + 8;  // LDS row pitch in T elements (144 B: 16-B aligned, banks spread)

template <typename TT, int BITS>
__global__ __launch_bounds__(256) void qmm_n_kernel(const uint32_t* __restrict__ w,
                                                    const uint16_t* __restrict__ scales,
                                                    const uint16_t* __restrict__ biases,
                                                    const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int m,
                                                    int n, int k, int gs_shift, int k_part,
                                                    float* __restrict__ partial) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[NT_M * NT_P];
  __shared__ __attribute__((aligned(16))) uint16_t wt[NT_N * NT_P];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * NT_M, n0 = blockIdx.x * NT_N;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;  // this wave's 32 x 32 quadrant
  const int r16 = lane & 15, g = lane >> 4;
  const size_t row_words = (size_t)n * BITS / 32;
  const int G = n >> gs_shift;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int k_lo = blockIdx.z * k_part, k_hi = min(k, k_lo + k_part);  // k_part % NT_K == 0
  // Raw inputs of one K-step, loaded a step ahead: two 8-k activation pieces
  // per thread, and for threads < 128 one 32-column weight chunk of one k row
  // with its (scale, bias).
  u32x4 xv[2];
  uint32_t wv[BITS];
  uint16_t sv = 0, bv = 0;
  const int kr = tid >> 1, c = tid & 1;
  const int col = n0 + 32 * c;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = tid + 256 * h;
      const int gm = m0 + (i >> 3), gk = k0 + 8 * (i & 7);
      xv[h] = u32x4{0u, 0u, 0u, 0u};
      if (gm < m && gk < k_hi) xv[h] = *reinterpret_cast<const u32x4*>(x + (size_t)gm * k + gk);
    }
    if (tid < 2 * NT_K) {
      const int gk = k0 + kr;
      if (gk < k_hi && col < n) {
        load_chunk<BITS>(w + (size_t)gk * row_words, (size_t)(col >> 5), wv);
        const size_t gi = (size_t)gk * G + (size_t)(col >> gs_shift);
        sv = scales[gi];
        bv = biases[gi];
      } else {
#pragma unroll
        for (int j = 0; j < BITS; ++j) wv[j] = 0u;
        sv = bv = 0;  // zero scale and bias: the chunk dequantizes to +0
      }
    }
  };
  if (k_lo < k_hi) fetch(k_lo);
  for (int k0 = k_lo; k0 < k_hi; k0 += NT_K) {
    // Stage the fetched step: activations as is, weights dequantized and
    // transposed into wt[n][k].
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = tid + 256 * h;
      *reinterpret_cast<u32x4*>(&xs[(i >> 3) * NT_P + 8 * (i & 7)]) = xv[h];
    }
    if (tid < 2 * NT_K) {
      uint32_t o[16];
      dequant_chunk<TT, BITS>(wv, TT::to_f32(sv), TT::to_f32(bv), o);
      uint16_t* dst = &wt[(32 * c) * NT_P + kr];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        dst[(2 * j) * NT_P] = (uint16_t)(o[j] & 0xffffu);
        dst[(2 * j + 1) * NT_P] = (uint16_t)(o[j] >> 16);
      }
    }
    if (k0 + NT_K < k_hi) fetch(k0 + NT_K);  // in flight during the MFMAs
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < NT_K; ks += 32) {
      u32x4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const u32x4*>(&xs[(wm + 16 * i + r16) * NT_P + ks + 8 * g]);
        b[i] = *reinterpret_cast<const u32x4*>(&wt[(wn + 16 * i + r16) * NT_P + ks + 8 * g]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = Mfma16<TT>::run(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  // D layout: lane (column r16, group g) holds rows 4g .. 4g+3 of a 16 x 16 block.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn + 16 * j + r16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm + 16 * i + 4 * g + e;
        if (row < m && col < n) {
          if (partial)
            partial[((size_t)blockIdx.z * m + row) * n + col] = acc[i][j][e];
          else
            y[(size_t)row * n + col] = TT::from_f32(acc[i][j][e]);
        }
      }
    }
}

// y = RNE_T(sum over parts p in order of partial[p]).
template <typename TT>
__global__ __launch_bounds__(256) void qmm_n_reduce_kernel(const float* __restrict__ partial, int parts, size_t mn,
                                                           uint16_t* __restrict__ y) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += stride) {
    float v = partial[i];
    for (int p = 1; p < parts; ++p) v += partial[(size_t)p * mn + i];
    y[i] = TT::from_f32(v);
  }
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                    float* partial) {
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  const int k_part = split > 1 ? (k / split + NT_K - 1) / NT_K * NT_K : (k + NT_K - 1) / NT_K * NT_K;
  const int parts = split > 1 ? (k + k_part - 1) / k_part : 1;
  const dim3 grid((unsigned)((n + NT_N - 1) / NT_N), (unsigned)((m + NT_M - 1) / NT_M), (unsigned)parts);
  hipLaunchKernelGGL((qmm_n_kernel<TT, BITS>), grid, dim3(256), 0, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), m, n, k, gs_shift, k_part > 0 ? k_part : NT_K,
                     parts > 1 ? partial : nullptr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || parts <= 1) return e;
  const size_t mn = (size_t)m * n;
  size_t blocks = (mn + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  hipLaunchKernelGGL((qmm_n_reduce_kernel<TT>), dim3((unsigned)blocks), dim3(256), 0, s, partial, parts, mn,
                     static_cast<uint16_t*>(y));
  return hipGetLastError();
}

template <typename TT>
hipError_t launch_bits(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                       float* partial) {
  switch (q.bits) {
    case 2: return launch_t<TT, 2>(s, q, x, y, m, n, k, split, partial);
    case 3: return launch_t<TT, 3>(s, q, x, y, m, n, k, split, partial);
    case 4: return launch_t<TT, 4>(s, q, x, y, m, n, k, split, partial);
    case 5: return launch_t<TT, 5>(s, q, x, y, m, n, k, split, partial);
    case 6: return launch_t<TT, 6>(s, q, x, y, m, n, k, split, partial);
    case 8: return launch_t<TT, 8>(s, q, x, y, m, n, k, split, partial);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// Parts of K so that the grid has about two workgroups per CU, each part at
// least two 64-deep K steps.
int qmm_n_split(int m, int n, int k, int cu_count) {
  const long tiles = (long)((n + NT_N - 1) / NT_N) * ((m + NT_M - 1) / NT_M);
  const long want = 2L * (cu_count > 0 ? cu_count : 256);
  int split = 1;
  while (tiles * split * 2 <= want && k / (split * 2) >= 2 * NT_K) split *= 2;
  return split;
}

size_t qmm_n_scratch_bytes(int m, int n, int split) { return split > 1 ? (size_t)split * m * n * 4 : 0; }

hipError_t launch_qmm_n(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                        float* partial) {
  if (m == 0 || n == 0) return hipSuccess;  // K == 0 still runs: it stores zeros
  if (split > 1 && !partial) return hipErrorInvalidValue;
  if (q.dtype == CPQ_DTYPE_BF16) return launch_bits<BF16>(s, q, x, y, m, n, k, split, partial);
  if (q.dtype == CPQ_DTYPE_F16) return launch_bits<F16>(s, q, x, y, m, n, k, split, partial);
  return hipErrorInvalidValue;
}

}  // namespace cpq
