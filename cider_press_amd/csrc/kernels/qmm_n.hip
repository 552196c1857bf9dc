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
#include <algorithm>

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
// K: thread (chunk c = tid % 8, row slot r = tid / 8) takes rows
// k0 + r + 32 j (j < RPT) of each 32*RPT-row step of the part and issues
// all of their loads before any arithmetic: per row the 32-column chunk c
// (16 bytes at 4-bit; the 8 threads of a row slot read 128 contiguous bytes),
// its (scale, bias) word and x[k].  Each column's weights of two rows are
// rounded to a T pair along k by one convert and accumulated with one v_dot2
// (products of two T exact in fp32).  The (scale, bias) of row k is
// element k * G + group of the flat tables; it is read as the aligned 4-byte
// word holding it (G may be odd).  Rows past the part take x = 0 and zero
// constants (exact zeros).  The 32 row slots are added through LDS in slot
// order.  With K split over parts the parts meet in the session scratch:
// each stores its 256 sums with the sc1 policy (written through to the
// memory side), waits until every store is acknowledged and only then
// counts its arrival on the column block's counter; the last arriver (the
// count it read is parts - 1) therefore finds every other part complete,
// loads their sums with sc1, adds the parts in part order and clears the
// counter for the next launch.
// ---------------------------------------------------------------------------
constexpr int QV_COLS = 256, QV_SLOTS = 32, QV_MAX_PARTS = 64;
constexpr int kQvMaxWords = 6144;  // column blocks * parts with K split (counters of blocks < 4096)

__device__ __forceinline__ uint32_t half_of(uint32_t word, uint32_t hi) { return hi ? word >> 16 : word & 0xffffu; }

// Columns 8P .. 8P+7 of a chunk as fp32 fmaf(s, q, b) (not yet rounded to T).
template <int BITS, int P>
__device__ __forceinline__ void dequant8_f32(const uint32_t* w, float s, float s16, float b, float* out) {
  if constexpr (BITS == 4) {
    // lo bytes = even nibbles q, hi bytes = odd nibbles as 16*q; s16*(16q) == s*q exactly.
    const uint32_t lo = opaque(w[P] & 0x0F0F0F0Fu);
    const uint32_t hi = opaque(w[P] & 0xF0F0F0F0u);
    out[0] = fmaf(s, ubyte_f32<0>(lo), b); out[1] = fmaf(s16, ubyte_f32<0>(hi), b);
    out[2] = fmaf(s, ubyte_f32<1>(lo), b); out[3] = fmaf(s16, ubyte_f32<1>(hi), b);
    out[4] = fmaf(s, ubyte_f32<2>(lo), b); out[5] = fmaf(s16, ubyte_f32<2>(hi), b);
    out[6] = fmaf(s, ubyte_f32<3>(lo), b); out[7] = fmaf(s16, ubyte_f32<3>(hi), b);
  } else {
    static_assert(BITS == 8, "4- and 8-bit only");
    const uint32_t w0 = w[2 * P], w1 = w[2 * P + 1];
    out[0] = fmaf(s, ubyte_f32<0>(w0), b); out[1] = fmaf(s, ubyte_f32<1>(w0), b);
    out[2] = fmaf(s, ubyte_f32<2>(w0), b); out[3] = fmaf(s, ubyte_f32<3>(w0), b);
    out[4] = fmaf(s, ubyte_f32<0>(w1), b); out[5] = fmaf(s, ubyte_f32<1>(w1), b);
    out[6] = fmaf(s, ubyte_f32<2>(w1), b); out[7] = fmaf(s, ubyte_f32<3>(w1), b);
  }
}

// Sum of the parts' values for column tid in part order, own part `mine`
// from a register, the others loaded with the sc1 policy, all NP loads in
// flight at once (a slot past `parts` re-reads part 0 and is not added).
template <int NP>
__device__ __forceinline__ float qv_sum_parts(__amdgpu_buffer_rsrc_t pr, int parts, int kp, int tid, float mine) {
  float pv[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int kk = i < parts ? i : 0;
    pv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, (uint32_t)(kk * QV_COLS + tid) * 4u, 0,
                                                                          16 /* sc1 */));
  }
  float sum = kp == 0 ? mine : pv[0];
#pragma unroll
  for (int i = 1; i < NP; ++i)
    if (i < parts) sum += i == kp ? mine : pv[i];
  return sum;
}

// Arrival counter of column block b: 128 bytes apart (distinct for b < 4096).
__device__ __forceinline__ int qv_counter(int b) { return (b & 127) * 32 + (b >> 7); }

template <typename TT, int BITS, int RPT>
__global__ __launch_bounds__(256) void qvm_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ y, int n, int k, int gs_shift, int k_part,
                                                  float* __restrict__ partial, unsigned int* __restrict__ counters) {
  static_assert(RPT % 2 == 0, "rows are taken two at a time");
  __shared__ float red[QV_SLOTS][QV_COLS + 4];
  __shared__ unsigned int arrived;
  const int tid = threadIdx.x;
  const int c = tid & 7, rs = tid >> 3;
  const int n0 = blockIdx.x * QV_COLS;
  const int chunk = min((n0 >> 5) + c, (n >> 5) - 1);  // columns past N re-read the last chunk (not stored)
  const uint32_t G = (uint32_t)(n >> gs_shift);
  const uint32_t grp = (uint32_t)((chunk << 5) >> gs_shift);
  const uint32_t row_bytes = (uint32_t)n * BITS / 8;
  const int kp = blockIdx.y, parts = gridDim.y;
  const int k_lo = kp * k_part, k_hi = min(k, k_lo + k_part);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)k * row_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)scales, 0, (int)((uint32_t)k * G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)biases, 0, (int)((uint32_t)k * G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)k * 2u), 0x00020000);
  const uint32_t woff = (uint32_t)chunk * BITS * 4u;

  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
  for (int k0 = k_lo; k0 < k_hi; k0 += RPT * QV_SLOTS) {
    // Every load of the step first: RPT rows' weights, constants and x.
    uint32_t wv[RPT][BITS], sw[RPT], bw[RPT], xw[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int kr = k0 + rs + QV_SLOTS * j;
      const uint32_t krc = (uint32_t)(kr < k_hi ? kr : k_lo);  // a row past the part re-reads k_lo (zeroed below)
      const uint32_t wro = woff + krc * row_bytes;  // per row slot: in the per-lane offset
#pragma unroll
      for (int q = 0; q < BITS / 4; ++q) {
        const u32x4 v4 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wro + 16u * q, 0, 0));
        wv[j][4 * q] = v4.x; wv[j][4 * q + 1] = v4.y; wv[j][4 * q + 2] = v4.z; wv[j][4 * q + 3] = v4.w;
      }
      const uint32_t e = krc * G + grp;
      sw[j] = __builtin_amdgcn_raw_buffer_load_b32(sr, (e & ~1u) * 2u, 0, 0);
      bw[j] = __builtin_amdgcn_raw_buffer_load_b32(br, (e & ~1u) * 2u, 0, 0);
      xw[j] = __builtin_amdgcn_raw_buffer_load_b32(xr, (krc & ~1u) * 2u, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < RPT; j += 2) {
      const int ka = k0 + rs + QV_SLOTS * j, kb = ka + QV_SLOTS;
      const bool la = ka < k_hi, lb = kb < k_hi;
      const uint32_t kac = (uint32_t)(la ? ka : k_lo), kbc = (uint32_t)(lb ? kb : k_lo);
      const uint32_t ea = kac * G + grp, eb = kbc * G + grp;
      const float sa = la ? TT::to_f32((uint16_t)half_of(sw[j], ea & 1u)) : 0.f;
      const float ba = la ? TT::to_f32((uint16_t)half_of(bw[j], ea & 1u)) : 0.f;
      const float sb = lb ? TT::to_f32((uint16_t)half_of(sw[j + 1], eb & 1u)) : 0.f;
      const float bb = lb ? TT::to_f32((uint16_t)half_of(bw[j + 1], eb & 1u)) : 0.f;
      const uint32_t xa = la ? half_of(xw[j], kac & 1u) : 0u;
      const uint32_t xb = lb ? half_of(xw[j + 1], kbc & 1u) : 0u;
      const uint32_t xab = xa | (xb << 16);  // (x[ka], x[kb]) as a T pair
#pragma unroll
      for (int p = 0; p < 4; ++p) {  // 8 columns 8p .. 8p+7 of the chunk
        float fa[8], fb[8];
        dequant8_f32<BITS, 0>(BITS == 4 ? &wv[j][p] : &wv[j][2 * p], sa, sa * 0.0625f, ba, fa);
        dequant8_f32<BITS, 0>(BITS == 4 ? &wv[j + 1][p] : &wv[j + 1][2 * p], sb, sb * 0.0625f, bb, fb);
#pragma unroll
        for (int i = 0; i < 8; ++i)  // (w[ka][n], w[kb][n]) rounded to T, n = 8p + i
          acc[8 * p + i] = TT::dot2(TT::pack2(fa[i], fb[i]), xab, acc[8 * p + i]);
      }
    }
  }

  // Row slots in order: this part's sum for column n0 + tid.
#pragma unroll
  for (int i = 0; i < 32; ++i) red[rs][32 * c + i] = acc[i];
  __syncthreads();
  float v = red[0][tid];
#pragma unroll
  for (int r = 1; r < QV_SLOTS; ++r) v += red[r][tid];

  if (parts > 1) {
    constexpr int SC1 = 16;
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(partial + (size_t)blockIdx.x * parts * QV_COLS), 0, parts * QV_COLS * 4, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), pr, (uint32_t)(kp * QV_COLS + tid) * 4u, 0,
                                          SC1);
    // Arrive only once every thread's store is acknowledged by the memory
    // side: the last arriver then reads every part without waiting.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      arrived = __hip_atomic_fetch_add(&counters[qv_counter(blockIdx.x)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != (unsigned int)(parts - 1)) return;
    v = parts <= 16   ? qv_sum_parts<16>(pr, parts, kp, tid, v)
        : parts <= 32 ? qv_sum_parts<32>(pr, parts, kp, tid, v)
                      : qv_sum_parts<QV_MAX_PARTS>(pr, parts, kp, tid, v);
    if (tid == 0) __hip_atomic_store(&counters[qv_counter(blockIdx.x)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const int col = n0 + tid;
  if (col < n) y[col] = TT::from_f32(v);
}

template <typename TT, int BITS, int RPT>
hipError_t launch_qvm_t(hipStream_t s, const QvmPlan& p, void* scratch, const QuantArgs& q, const void* x, void* y,
                        int n, int k) {
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  const dim3 grid((unsigned)((n + QV_COLS - 1) / QV_COLS), (unsigned)p.parts);
  unsigned int* counters = p.parts > 1 ? static_cast<unsigned int*>(scratch) : nullptr;
  float* partial =
      p.parts > 1 ? reinterpret_cast<float*>(static_cast<char*>(scratch) + kWideCounterBytes) : nullptr;
  hipLaunchKernelGGL((qvm_kernel<TT, BITS, RPT>), grid, dim3(256), 0, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), n, k, gs_shift, p.k_part, partial, counters);
  return hipGetLastError();
}

template <typename TT, int BITS>
hipError_t launch_qvm_rpt(hipStream_t s, const QvmPlan& p, void* scratch, const QuantArgs& q, const void* x, void* y,
                          int n, int k) {
  switch (p.rpt) {
    case 2: return launch_qvm_t<TT, BITS, 2>(s, p, scratch, q, x, y, n, k);
    case 4: return launch_qvm_t<TT, BITS, 4>(s, p, scratch, q, x, y, n, k);
    default: return hipErrorInvalidValue;
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

// The decode kernel's plan: rows per thread and step (4; 2 when the
// 4-row steps number more than four per CU, where shorter steps in a loop
// measured faster: N = 12288 and K = 14336 at N = 4096), then K parts
// (whole steps) until the grid has about four workgroups per CU, at most
// 64 parts.  Parts need the arrival words and 1 KiB of fp32 sums per
// (column block, part); without that much session scratch, one part.
QvmPlan qvm_plan(const QuantArgs& q, int n, int k, int cu_count, size_t scratch_cap) {
  const long cus = cu_count > 0 ? cu_count : 256;
  const long blocks = (n + QV_COLS - 1) / QV_COLS;
  int rpt = blocks * ((k + 4 * QV_SLOTS - 1) / (4 * QV_SLOTS)) > 4 * cus ? 2 : 4;
  rpt = env_int("CPQ_QVM_RPT", rpt);
  if (rpt != 2 && rpt != 4) rpt = 4;
  const long step = (long)rpt * QV_SLOTS;
  const long steps = (k + step - 1) / step;
  long parts = std::min<long>({steps, (long)QV_MAX_PARTS, std::max<long>(1, 4 * cus / blocks)});
  parts = std::min<long>(parts, std::max<long>(1, kQvMaxWords / blocks));
  const int forced = env_int("CPQ_QVM_PARTS", 0);
  if (forced > 0) parts = std::min<long>({(long)forced, steps, (long)QV_MAX_PARTS, std::max<long>(1, kQvMaxWords / blocks)});
  long k_part = (steps + parts - 1) / parts * step;
  parts = (k + k_part - 1) / k_part;
  size_t bytes = parts > 1 ? kWideCounterBytes + (size_t)blocks * parts * QV_COLS * 4 : 0;
  if (bytes > scratch_cap) {
    parts = 1;
    k_part = steps * step;
    bytes = 0;
  }
  return QvmPlan{rpt, (int)parts, (int)k_part, bytes};
}

bool qvm_fits(const QuantArgs& q, int n, int k) {
  if (q.bits != 4 && q.bits != 8) return false;
  if (q.dtype != CPQ_DTYPE_BF16 && q.dtype != CPQ_DTYPE_F16) return false;
  if (n % 32 != 0 || k < 1) return false;
  if ((uint64_t)k * (uint64_t)n * q.bits / 8 >= (1ull << 31)) return false;
  if ((uint64_t)k * (uint64_t)(n / q.gs) * 2 >= (1ull << 31)) return false;
  // 16-byte weight loads, 4-byte scale/bias and x words.
  return (reinterpret_cast<uintptr_t>(q.w) & 15u) == 0 &&
         ((reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases)) & 3u) == 0;
}

hipError_t launch_qvm(hipStream_t s, const QvmPlan& p, void* scratch, const QuantArgs& q, const void* x, void* y,
                      int n, int k) {
  if (p.parts > 1 && !scratch) return hipErrorInvalidValue;
  if (p.parts < 1 || p.parts > QV_MAX_PARTS || (long)((n + QV_COLS - 1) / QV_COLS) * p.parts > kQvMaxWords ||
      (long)p.k_part * p.parts < k)
    return hipErrorInvalidValue;
  if (q.dtype == CPQ_DTYPE_BF16)
    return q.bits == 4 ? launch_qvm_rpt<BF16, 4>(s, p, scratch, q, x, y, n, k)
                       : launch_qvm_rpt<BF16, 8>(s, p, scratch, q, x, y, n, k);
  if (q.dtype == CPQ_DTYPE_F16)
    return q.bits == 4 ? launch_qvm_rpt<F16, 4>(s, p, scratch, q, x, y, n, k)
                       : launch_qvm_rpt<F16, 8>(s, p, scratch, q, x, y, n, k);
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
