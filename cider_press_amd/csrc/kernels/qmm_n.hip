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

// ---------------------------------------------------------------------------
// Decode (M = 1) at 4 and 8 bits: y[n] = sum_k x[k] * RNE_T(fmaf(s, q, b))
// on the VALU.  A workgroup (256 threads) owns 256 columns and one part of
// K: thread (chunk c = tid % 8, row slot r = tid / 8) walks rows
// k = k_lo + r, k_lo + r + 32, ... of the part, two rows at a time; per row
// it reads the 32-column chunk c (one 16-byte load at 4-bit, the 8 threads of
// a row slot reading 128 contiguous bytes) and its (scale, bias) word.  The
// two rows' dequantized pairs (along n) are regrouped into pairs along k and
// accumulated with one v_dot2 per two weights (products of two T exact in
// fp32).  The (scale, bias) of row k is element k * G + group of the flat
// tables; it is read as the aligned 4-byte word holding it (G may be odd).  The 32 row slots are then added through LDS in slot order; with
// K split over parts, each part stores fp32 partial sums that
// qmm_n_reduce_kernel adds in part order.  Rows past K, or past the part,
// take x = 0 and zero constants (exact zeros).
// ---------------------------------------------------------------------------
constexpr int QV_COLS = 256, QV_SLOTS = 32;

template <typename TT, int BITS>
__global__ __launch_bounds__(256) void qvm_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ y, int n, int k, int gs_shift, int k_part,
                                                  float* __restrict__ partial) {
  __shared__ float red[QV_SLOTS][QV_COLS + 4];
  const int tid = threadIdx.x;
  const int c = tid & 7, rs = tid >> 3;
  const int n0 = blockIdx.x * QV_COLS;
  const int chunk = min((n0 >> 5) + c, (n >> 5) - 1);  // columns past N re-read the last chunk (not stored)
  const int G = n >> gs_shift;
  const int grp = (chunk << 5) >> gs_shift;
  const uint32_t row_words = (uint32_t)n * BITS / 32;
  const int k_lo = blockIdx.y * k_part, k_hi = min(k, k_lo + k_part);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)k * row_words * 4u), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)scales, 0, (int)((uint32_t)k * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)biases, 0, (int)((uint32_t)k * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)k * 2u), 0x00020000);
  const uint32_t woff = (uint32_t)chunk * BITS * 4u;

  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
  // Two rows per step: ka = k_lo + rs + 64 j, kb = ka + 32.
  for (int ka = k_lo + rs; ka < k_hi; ka += 2 * QV_SLOTS) {
    const int kb = ka + QV_SLOTS;
    const bool lb = kb < k_hi;
    const int kbc = lb ? kb : ka;  // a row past the part re-reads row ka (zeroed below)
    // Row offsets differ per row slot: they go into the per-lane offset.
    const uint32_t wra = woff + (uint32_t)ka * row_words * 4u, wrb = woff + (uint32_t)kbc * row_words * 4u;
    uint32_t wa[BITS], wb[BITS];
#pragma unroll
    for (int q = 0; q < BITS / 4; ++q) {
      const u32x4 va = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wra + 16u * q, 0, 0));
      const u32x4 vb = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wrb + 16u * q, 0, 0));
      wa[4 * q] = va.x; wa[4 * q + 1] = va.y; wa[4 * q + 2] = va.z; wa[4 * q + 3] = va.w;
      wb[4 * q] = vb.x; wb[4 * q + 1] = vb.y; wb[4 * q + 2] = vb.z; wb[4 * q + 3] = vb.w;
    }
    const uint32_t ea = (uint32_t)ka * (uint32_t)G + (uint32_t)grp, eb = (uint32_t)kbc * (uint32_t)G + (uint32_t)grp;
    const uint32_t swa = __builtin_amdgcn_raw_buffer_load_b32(sr, (ea & ~1u) * 2u, 0, 0);
    const uint32_t bwa = __builtin_amdgcn_raw_buffer_load_b32(br, (ea & ~1u) * 2u, 0, 0);
    const uint32_t swb = __builtin_amdgcn_raw_buffer_load_b32(sr, (eb & ~1u) * 2u, 0, 0);
    const uint32_t bwb = __builtin_amdgcn_raw_buffer_load_b32(br, (eb & ~1u) * 2u, 0, 0);
    const bool ha = (ea & 1u) != 0, hb = (eb & 1u) != 0;
    const uint32_t xwa = __builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)(ka & ~1) * 2u, 0, 0);
    const uint32_t xwb = __builtin_amdgcn_raw_buffer_load_b32(xr, (uint32_t)(kbc & ~1) * 2u, 0, 0);
    const float sa = TT::to_f32((uint16_t)(ha ? swa >> 16 : swa & 0xffffu));
    const float ba = TT::to_f32((uint16_t)(ha ? bwa >> 16 : bwa & 0xffffu));
    const float sb = lb ? TT::to_f32((uint16_t)(hb ? swb >> 16 : swb & 0xffffu)) : 0.f;
    const float bb = lb ? TT::to_f32((uint16_t)(hb ? bwb >> 16 : bwb & 0xffffu)) : 0.f;
    const uint32_t xa = (ka & 1) ? xwa >> 16 : xwa & 0xffffu;
    const uint32_t xb = lb ? ((kb & 1) ? xwb >> 16 : xwb & 0xffffu) : 0u;
    const uint32_t xab = xa | (xb << 16);  // (x[ka], x[kb]) as a T pair
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // 8 columns 8p .. 8p+7 of the chunk
      uint32_t ua[4], ub[4];
      dequant8<TT, BITS, 0>(BITS == 4 ? &wa[p] : &wa[2 * p], sa, sa * 0.0625f, ba, ua);
      dequant8<TT, BITS, 0>(BITS == 4 ? &wb[p] : &wb[2 * p], sb, sb * 0.0625f, bb, ub);
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // ua[i] = (w[ka][n], w[ka][n+1]), n = 8p + 2i
        const uint32_t lo = __builtin_amdgcn_perm(ub[i], ua[i], 0x05040100u);  // (w[ka][n], w[kb][n])
        const uint32_t hi = __builtin_amdgcn_perm(ub[i], ua[i], 0x07060302u);  // (w[ka][n+1], w[kb][n+1])
        acc[8 * p + 2 * i] = TT::dot2(lo, xab, acc[8 * p + 2 * i]);
        acc[8 * p + 2 * i + 1] = TT::dot2(hi, xab, acc[8 * p + 2 * i + 1]);
      }
    }
  }

  // Row slots in order, then one part's sum per column.
#pragma unroll
  for (int i = 0; i < 32; ++i) red[rs][32 * c + i] = acc[i];
  __syncthreads();
  const int col = n0 + tid;
  if (col < n) {
    float v = red[0][tid];
#pragma unroll
    for (int r = 1; r < QV_SLOTS; ++r) v += red[r][tid];
    if (partial)
      partial[(size_t)blockIdx.y * n + col] = v;
    else
      y[col] = TT::from_f32(v);
  }
}

template <typename TT, int BITS>
hipError_t launch_qvm_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k, int parts,
                        float* partial) {
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  const int k_part = (k + parts - 1) / parts;
  const int np = (k + k_part - 1) / k_part;
  const dim3 grid((unsigned)((n + QV_COLS - 1) / QV_COLS), (unsigned)np);
  hipLaunchKernelGGL((qvm_kernel<TT, BITS>), grid, dim3(256), 0, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), n, k, gs_shift, k_part, np > 1 ? partial : nullptr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || np <= 1) return e;
  size_t blocks = ((size_t)n + 255) / 256;
  hipLaunchKernelGGL((qmm_n_reduce_kernel<TT>), dim3((unsigned)blocks), dim3(256), 0, s, partial, np, (size_t)n,
                     static_cast<uint16_t*>(y));
  return hipGetLastError();
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

// The decode kernel's K parts: about two workgroups per CU, each part at
// least 256 rows (so the fixed per-workgroup work stays small next to it).
int qvm_parts(int n, int k, int cu_count) {
  const long blocks = (n + QV_COLS - 1) / QV_COLS;
  const long want = 2L * (cu_count > 0 ? cu_count : 256);
  int parts = 1;
  while (blocks * parts * 2 <= want && k / (parts * 2) >= 256) parts *= 2;
  return parts;
}

bool qvm_fits(const QuantArgs& q, int n, int k) {
  if (q.bits != 4 && q.bits != 8) return false;
  if (n % 32 != 0 || k < 1) return false;
  if ((uint64_t)k * (uint64_t)n * q.bits / 8 >= (1ull << 31)) return false;
  if ((uint64_t)k * (uint64_t)(n / q.gs) * 2 >= (1ull << 31)) return false;
  // 16-byte weight loads, 4-byte scale/bias and x words.
  return (reinterpret_cast<uintptr_t>(q.w) & 15u) == 0 &&
         ((reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases)) & 3u) == 0;
}

hipError_t launch_qvm(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k, int parts,
                      float* partial) {
  if (parts > 1 && !partial) return hipErrorInvalidValue;
  if (q.dtype == CPQ_DTYPE_BF16)
    return q.bits == 4 ? launch_qvm_t<BF16, 4>(s, q, x, y, n, k, parts, partial)
                       : launch_qvm_t<BF16, 8>(s, q, x, y, n, k, parts, partial);
  if (q.dtype == CPQ_DTYPE_F16)
    return q.bits == 4 ? launch_qvm_t<F16, 4>(s, q, x, y, n, k, parts, partial)
                       : launch_qvm_t<F16, 8>(s, q, x, y, n, k, parts, partial);
  return hipErrorInvalidValue;
}

hipError_t launch_qmm_n(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                        float* partial) {
  if (m == 0 || n == 0) return hipSuccess;  // K == 0 still runs: it stores zeros
  if (split > 1 && !partial) return hipErrorInvalidValue;
  if (q.dtype == CPQ_DTYPE_BF16) return launch_bits<BF16>(s, q, x, y, m, n, k, split, partial);
  if (q.dtype == CPQ_DTYPE_F16) return launch_bits<F16>(s, q, x, y, m, n, k, split, partial);
  return hipErrorInvalidValue;
}

}  // namespace cpq
