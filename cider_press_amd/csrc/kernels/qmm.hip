// Prefill quantized GEMM for gfx950: Y[M,N] = X[M,K] . dequant(W[N,K])^T.
//
// Reference op: affine_qmm_t / qmm_t_impl (kernels-mlx/.../quantized.h:1087-1213,
// 1713-1784), dispatched by crates/cider-press-kernels/src/kernels/qmm.rs:66-220.
// Same numerics: each W tile is dequantized to T (RNE of fmaf(s, q, b)) into
// LDS, multiplied on the matrix cores with fp32 accumulation, stored as T.
//
// Tiling: a 256-thread workgroup owns a BM x BN output tile and walks K in
// 32-element steps (one quantization chunk per W row, always inside one
// group).  Per step it stages the BM x 32 activation tile and the BN x 32
// dequantized weight tile in LDS (rows padded by 8 elements to spread banks),
// then each of the 4 waves (WM x WN arrangement) runs
// v_mfma_f32_32x32x16_{bf16,f16} on its (BM/WM) x (BN/WN) sub-tile, reading
// both operands with ds_read_b128.  Two LDS buffers alternate so the next
// step's global loads and dequantization overlap the current step's MFMAs.
// MFMA 32x32x16 operand layout: A[m][k] in lane m + 32*(k/8), element k%8;
// B[k][n] in lane n + 32*(k/8), element k%8; D[m][n] in lane n + 32*((m/4)%2),
// register 4*(m/8) + m%4.
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

template <typename TT>
struct Mfma32;
template <>
struct Mfma32<BF16> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma32<F16> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

constexpr int BK = 32;
constexpr int LDP = BK + 8;  // padded LDS row pitch (elements)

template <typename TT, int BITS, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void qmm_kernel(const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases,
                                                  const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ y, int m, int n, int k,
                                                  int gs_shift) {
  static_assert(WM * WN == 4, "4 waves per workgroup");
  constexpr int TM = BM / WM / 32;  // 32x32 blocks per wave along M
  constexpr int TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold whole 32x32 blocks");
  constexpr int XPIECES = BM * (BK / 8);  // 16-byte pieces of the X tile
  static_assert(BN <= 256, "one W row per thread");

  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][BM * LDP];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * LDP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int row0 = blockIdx.y * BM;
  const int col0 = blockIdx.x * BN;
  const int chunks = k >> 5;
  const size_t words_per_row = (size_t)k * BITS / 32;
  const int groups_per_row = k >> gs_shift;

  // This thread's W row (if any) and its base pointers.
  const int wr = tid;
  const bool w_ok = wr < BN && col0 + wr < n;
  const uint32_t* wrow = w + (size_t)(w_ok ? col0 + wr : 0) * words_per_row;
  const uint16_t* srow = scales + (size_t)(w_ok ? col0 + wr : 0) * groups_per_row;
  const uint16_t* brow = biases + (size_t)(w_ok ? col0 + wr : 0) * groups_per_row;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Register staging for the next K step.
  constexpr int XPER = (XPIECES + 255) / 256;
  u32x4 xreg[XPER];
  uint32_t wreg[BITS];
  float s_next = 0.f, b_next = 0.f;

  auto fetch = [&](int kc) {
#pragma unroll
    for (int p = 0; p < XPER; ++p) {
      const int piece = tid + 256 * p;
      xreg[p] = u32x4{0u, 0u, 0u, 0u};
      if (piece < XPIECES) {
        const int r = piece / (BK / 8);
        const int part = piece % (BK / 8);
        const int gm = row0 + r;
        if (gm < m)
          xreg[p] = *reinterpret_cast<const u32x4*>(x + (size_t)gm * k + (size_t)kc * 32 + part * 8);
      }
    }
    if (w_ok) {
      load_chunk<BITS>(wrow, (size_t)kc, wreg);
      const int gi = (kc << 5) >> gs_shift;
      s_next = TT::to_f32(srow[gi]);
      b_next = TT::to_f32(brow[gi]);
    }
  };

  auto stage = [&](int buf) {
#pragma unroll
    for (int p = 0; p < XPER; ++p) {
      const int piece = tid + 256 * p;
      if (piece < XPIECES) {
        const int r = piece / (BK / 8);
        const int part = piece % (BK / 8);
        *reinterpret_cast<u32x4*>(&Xs[buf][r * LDP + part * 8]) = xreg[p];
      }
    }
    if (wr < BN) {
      uint32_t o[16];
      if (w_ok) {
        dequant_chunk<TT, BITS>(wreg, s_next, b_next, o);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = 0u;
      }
      u32x4* dst = reinterpret_cast<u32x4*>(&Ws[buf][wr * LDP]);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
    }
  };

  fetch(0);
  stage(0);
  __syncthreads();

  const int arow = wm * (BM / WM) + (lane & 31);
  const int brow_l = wn * (BN / WN) + (lane & 31);
  const int koff = 8 * (lane >> 5);

  for (int kc = 0; kc < chunks; ++kc) {
    const int buf = kc & 1;
    const bool more = kc + 1 < chunks;
    if (more) fetch(kc + 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const u32x4*>(&Xs[buf][(arow + 32 * i) * LDP + 16 * kk + koff]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const u32x4*>(&Ws[buf][(brow_l + 32 * j) * LDP + 16 * kk + koff]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma32<TT>::run(a[i], b[j], acc[i][j]);
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: D[m][n] lives in lane n + 32*((m/4)%2), register 4*(m/8) + m%4.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int gcol = col0 + wn * (BN / WN) + 32 * j + (lane & 31);
      if (gcol >= n) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int grow = row0 + wm * (BM / WM) + 32 * i + r;
        if (grow < m) y[(size_t)grow * n + gcol] = TT::from_f32(acc[i][j][e]);
      }
    }
  }
}

int shift_of(int gs) {
  int s = 0;
  while ((1 << s) < gs) ++s;
  return s;
}

template <typename TT, int BITS, int BM, int BN, int WM, int WN>
hipError_t launch_cfg(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                      int k) {
  dim3 grid((unsigned)((n + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
  hipLaunchKernelGGL((qmm_kernel<TT, BITS, BM, BN, WM, WN>), grid, dim3(256), 0, s, q.w,
                     static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                     static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), m, n, k,
                     shift_of(q.gs));
  return hipGetLastError();
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  // Fill the chip: 128x128 tiles when they give at least ~2 workgroups per
  // CU, else 64-row tiles.
  const long tiles128 = (long)((m + 127) / 128) * ((n + 127) / 128);
  if (tiles128 >= 512) return launch_cfg<TT, BITS, 128, 128, 2, 2>(s, q, x, y, m, n, k);
  return launch_cfg<TT, BITS, 64, 128, 2, 2>(s, q, x, y, m, n, k);
}

}  // namespace

hipError_t launch_qmm(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                      int k) {
#define CPQ_QMM_BITS(TT)                                   \
  switch (q.bits) {                                        \
    case 2: return launch_t<TT, 2>(s, q, x, y, m, n, k);   \
    case 3: return launch_t<TT, 3>(s, q, x, y, m, n, k);   \
    case 4: return launch_t<TT, 4>(s, q, x, y, m, n, k);   \
    case 5: return launch_t<TT, 5>(s, q, x, y, m, n, k);   \
    case 6: return launch_t<TT, 6>(s, q, x, y, m, n, k);   \
    case 8: return launch_t<TT, 8>(s, q, x, y, m, n, k);   \
    default: return hipErrorInvalidValue;                  \
  }
  if (q.dtype == CPQ_DTYPE_BF16) { CPQ_QMM_BITS(BF16) }
  if (q.dtype == CPQ_DTYPE_F16) { CPQ_QMM_BITS(F16) }
#undef CPQ_QMM_BITS
  return hipErrorInvalidValue;
}

}  // namespace cpq
