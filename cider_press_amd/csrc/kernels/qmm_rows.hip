// Small-M quantized GEMM with the whole activation matrix resident in LDS:
// Y[M, N] = X[M, K] . dequant(W[N, K])^T for 1 <= M <= 64 rows whose
// activations fit in LDS (M * K * 2 bytes <= kRowsXMax), at any N, for the
// shapes where N is large and K short (a vocabulary projection at prefill:
// the reference's Qwen2.5-0.5B lm_head at M = 39 is N = 151936, K = 896).
//
// Reference semantics: qmm_t_impl (kernels-mlx/mlx/backend/metal/kernels/
// quantized.h:1087-1213): each weight is dequantized to T as
// RNE_T(fmaf(scale, q, bias)), products accumulate in fp32, the output is
// rounded to T once.
//
// HBM-bound: every weight is read and dequantized exactly once, and every
// dequantized 32-element slice feeds the MFMAs of all row blocks.
//   - workgroup = 8 waves = 128 columns; wave w owns the 16 columns
//     16 (8 blockIdx.x + w) and walks all of K in 128-element steps;
//   - the activation rows are copied into LDS once per workgroup by the
//     buffer-to-LDS path (no VGPRs, natural element order): slot j of step t
//     of row r holds 16-byte piece j ^ swz_key(r & 15) of that step, so the
//     16 lanes an operand read serves together hit 16 distinct slots;
//   - lane (column r, chunk group g) loads, per step, the 32-element chunk g
//     of its column (16 bytes at 4 bits) and its (scale, bias), and
//     dequantizes it slice by slice in natural order into the B operand of
//     v_mfma_f32_16x16x32 (B[k][n] in lane n + 16 (k / 8)); the A operand of
//     row block rb is rows 16 rb .. 16 rb + 15 (rows past M read row M-1,
//     never stored), D[m][n] in lane n + 16 (m / 4), element m % 4;
//   - batches of up to 8 steps (4 at 8 bits): each batch's (scale, bias)
//     loads, then its weight loads, issued in one straight run (the batch
//     body exists for 8, 4, 2 and 1 steps; slots past the batch read at an
//     offset past every range, which returns zeros), so a step's multiply
//     waits for its own weights only; a vote within the wave picks the
//     single-FMA dequantization for the batch.
#include <algorithm>
#include <type_traits>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int kRowsWaves = 8;               // waves per workgroup
constexpr int kRowsNCB = 1;                 // 16-column blocks per wave
constexpr int kRowsCols = 16 * kRowsNCB * kRowsWaves;  // columns per workgroup
constexpr int kRowsXMax = 78 * 1024;        // LDS bytes of the activation rows (two workgroups per CU)

__device__ __forceinline__ uint64_t rows_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

template <int BITS>
__device__ __forceinline__ void rows_load(__amdgpu_buffer_rsrc_t wr, uint32_t voff, uint32_t* dst) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, 0, 0));
  dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
  if constexpr (BITS == 8) {
    const u32x4 v1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff + 16, 0, 0));
    dst[4] = v1.x; dst[5] = v1.y; dst[6] = v1.z; dst[7] = v1.w;
  }
}

// One 128-k step of a wave: four 32-k slices; each slice of each column
// block is dequantized once, each row block's A operand is read once, and
// every (row block, column block) pair gets one MFMA.  xs: the step's
// 256-byte block of row 0 (row r at xs + r * rstride); rows[rb]: the clamped
// row of this lane's A operand in row block rb.
template <typename TT, int BITS, bool FAST, int RBK>
__device__ __forceinline__ void rows_step(const uint32_t (*wq)[BITS], const uint32_t* sv, const uint32_t* bv,
                                          const unsigned char* xs, int rstride, const int* rows,
                                          f32x4 (*acc)[kRowsNCB]) {
  float s[kRowsNCB], b[kRowsNCB], s16[kRowsNCB], c0[kRowsNCB], c1[kRowsNCB];
#pragma unroll
  for (int c = 0; c < kRowsNCB; ++c) {
    s[c] = TT::to_f32((uint16_t)sv[c]);
    b[c] = TT::to_f32((uint16_t)bv[c]);
    s16[c] = s[c] * 0.0625f;
    c0[c] = fmaf(-1024.f, s[c], b[c]);
    c1[c] = fmaf(-64.f, s[c], b[c]);
  }
  const int g = (threadIdx.x >> 4) & 3;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4 bo[kRowsNCB];
#pragma unroll
    for (int c = 0; c < kRowsNCB; ++c) {
      if (i == 0) bo[c] = dequant_slice_nat<TT, BITS, FAST, 0>(wq[c], s[c], s16[c], b[c], c0[c], c1[c]);
      if (i == 1) bo[c] = dequant_slice_nat<TT, BITS, FAST, 1>(wq[c], s[c], s16[c], b[c], c0[c], c1[c]);
      if (i == 2) bo[c] = dequant_slice_nat<TT, BITS, FAST, 2>(wq[c], s[c], s16[c], b[c], c0[c], c1[c]);
      if (i == 3) bo[c] = dequant_slice_nat<TT, BITS, FAST, 3>(wq[c], s[c], s16[c], b[c], c0[c], c1[c]);
    }
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb) {
      const int row = rows[rb];
      const u32x4 a =
          *reinterpret_cast<const u32x4*>(xs + row * rstride + (((4 * g + i) ^ swz_key(row & 15)) << 4));
#pragma unroll
      for (int c = 0; c < kRowsNCB; ++c) acc[rb][c] = Mfma16<TT>::run(a, bo[c], acc[rb][c]);
    }
  }
}

template <typename TT, int BITS, int RBK, bool WIDE>
__global__ __launch_bounds__(64 * kRowsWaves) __attribute__((amdgpu_waves_per_eu(BITS == 4 && RBK < 4 ? 4 : 3))) void qmm_rows_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int m, int n, int k, int gs_shift) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int PFMAX = (BITS == 4 ? 8 : 4) / kRowsNCB;  // steps per batch
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * kRowsWaves + wave) * (16 * kRowsNCB);
  const int S = k >> 7;          // steps of 128
  const int SPR = (S + 3) >> 2;  // 1 KiB copies per activation row (4 steps each)
  const int rstride = SPR * 1024;
  const int G = k >> gs_shift;
  const uint32_t rowbytes = (uint32_t)k * BITS / 8u;
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)scales, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)biases, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);

  // 1. Activation rows into LDS, row r at byte r * rstride: copy i (64 lanes
  //    x 16 bytes, at byte 1024 i) is row i / SPR, steps 4 (i % SPR) + g;
  //    lane (j, g) fills slot j of its step with piece j ^ swz_key(row & 15).  Steps
  //    past K read zeros (offset past the range) into the row's rounding.
  const int ncopies = m * SPR;
  for (int i = wave; i < ncopies; i += kRowsWaves) {
    const int row = i / SPR;
    const int t = 4 * (i - row * SPR) + g;
    const int pc = r ^ swz_key(row & 15);
    const uint32_t off =
        t < S ? ((uint32_t)row * (uint32_t)k + (uint32_t)t * 128u + (uint32_t)pc * 8u) * 2u : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(smem + 1024 * i), 16,
                                             off, 0, 0, 0);
  }
  // The first batch waits for the copies by count (wait_vmcnt below): no
  // load may move above them.
  __asm__ __volatile__("" ::: "memory");

  // 2. This lane's weight streams: columns n0 + 16 c + r, chunk g of each
  //    step.  Columns past N read zeros through the range check (offsets
  //    past 2^31, beyond every range; never stored).
  uint32_t voff0[kRowsNCB], coff0[kRowsNCB];
#pragma unroll
  for (int c = 0; c < kRowsNCB; ++c) {
    const int col = n0 + 16 * c + r;
    voff0[c] = col < n ? (uint32_t)col * rowbytes + (uint32_t)g * (BITS * 4u) : 0x80000000u;
    coff0[c] = col < n ? (uint32_t)col * (uint32_t)G : 0x40000000u;
  }
  int rows[RBK];
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb) rows[rb] = min(16 * rb + r, m - 1);
  f32x4 acc[RBK][kRowsNCB];
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
    for (int c = 0; c < kRowsNCB; ++c) acc[rb][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto batch = [&](int b0, int nb, auto pfc) {
    constexpr int PF = decltype(pfc)::value;
    uint32_t wq[PF][kRowsNCB][BITS];
    // (scale, bias) of each step.  WIDE (group size 64, an even number of
    // groups per row, so every column's row starts on a 32-bit word and K
    // is a multiple of 128): the column's words for the batch in one or two
    // 16-byte loads per table (word T holds step T's two groups; a 2-byte
    // load per step and value is what the routed-decode kernel measured
    // 3.3 us slower at 4 tokens), the lane's halves of steps t, t + 1 packed
    // into one register.  Otherwise a 16-bit load per step and value.
    constexpr int NP = WIDE ? (PF + 1) / 2 : PF;
    constexpr int NSB = WIDE ? (PF >= 4 ? PF / 4 : 1) : PF;  // loads per table
    uint32_t sv[NP][kRowsNCB], bv[NP][kRowsNCB];
    if constexpr (WIDE) {
      static_assert(kRowsNCB == 1, "one column block per wave");
      uint32_t sw[PF], bw[PF];
      const uint32_t wo = (coff0[0] + 2u * (uint32_t)b0) * 2u;  // past 2^31 for columns past N
      if constexpr (PF >= 4) {
#pragma unroll
        for (int q = 0; q < PF; q += 4) {
          const u32x4 s4 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, wo + 4u * q, 0, 0));
          const u32x4 b4 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(br, wo + 4u * q, 0, 0));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sw[q + i] = s4[i];
            bw[q + i] = b4[i];
          }
        }
      } else if constexpr (PF == 2) {
        const u32x2 s2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, wo, 0, 0));
        const u32x2 b2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(br, wo, 0, 0));
        sw[0] = s2[0];
        sw[1] = s2[1];
        bw[0] = b2[0];
        bw[1] = b2[1];
      } else {
        sw[0] = __builtin_amdgcn_raw_buffer_load_b32(sr, wo, 0, 0);
        bw[0] = __builtin_amdgcn_raw_buffer_load_b32(br, wo, 0, 0);
      }
      // Half g / 2 of words t and t + 1 into bits 0..15 and 16..31.
      const uint32_t psel = (g >> 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const int t1 = 2 * j + 1 < PF ? 2 * j + 1 : 2 * j;
        sv[j][0] = __builtin_amdgcn_perm(sw[t1], sw[2 * j], psel);
        bv[j][0] = __builtin_amdgcn_perm(bw[t1], bw[2 * j], psel);
      }
    } else {
#pragma unroll
      for (int t = 0; t < PF; ++t)
#pragma unroll
        for (int c = 0; c < kRowsNCB; ++c) {
          const uint32_t gi = coff0[c] + (((uint32_t)(4 * (b0 + t) + g) * 32u) >> gs_shift);
          const uint32_t so = t < nb ? gi * 2u : 0x80000000u;
          sv[t][c] = __builtin_amdgcn_raw_buffer_load_b16(sr, so, 0, 0);
          bv[t][c] = __builtin_amdgcn_raw_buffer_load_b16(br, so, 0, 0);
        }
    }
    // Step t's 16-bit scale / bias of column block c (bits 0..15).
    auto sval = [&](int t, int c) -> uint32_t {
      if constexpr (WIDE) return (t & 1) ? sv[t >> 1][c] >> 16 : sv[t >> 1][c] & 0xffffu;
      else return sv[t][c];
    };
    auto bval = [&](int t, int c) -> uint32_t {
      if constexpr (WIDE) return (t & 1) ? bv[t >> 1][c] >> 16 : bv[t >> 1][c] & 0xffffu;
      else return bv[t][c];
    };
#pragma unroll
    for (int t = 0; t < PF; ++t)
#pragma unroll
      for (int c = 0; c < kRowsNCB; ++c)
        rows_load<BITS>(wr, t < nb ? voff0[c] + (uint32_t)(b0 + t) * (16u * BITS) : 0x80000000u, wq[t][c]);
    if (b0 == 0) {
      // The activation copies are older than this batch's loads.
      wait_vmcnt<kRowsNCB * (2 * NSB + PF * (BITS / 4))>();
      __syncthreads();
    }
    // Vote: the packed exponent check over the batch's (scale, bias) pairs
    // (two per word; slots past the batch repeat the first pair), and the
    // exact per-group check only when some lane fails it.
    FastQuick fq;
    fast_quick_init(fq);
#pragma unroll
    for (int c = 0; c < kRowsNCB; ++c)
#pragma unroll
      for (int t = 0; t < PF; t += 2) {
        const int t1 = t + 1 < PF ? t + 1 : t;
        const uint32_t s0 = t < nb ? sval(t, c) : sval(0, c), b0v = t < nb ? bval(t, c) : bval(0, c);
        const uint32_t s1 = t1 < nb ? sval(t1, c) : sval(0, c), b1v = t1 < nb ? bval(t1, c) : bval(0, c);
        fast_quick_add<TT>(fq, s0 | (s1 << 16), b0v | (b1v << 16));
      }
    bool fast = rows_ballot(!fast_quick_ok<TT>(fq)) == 0;
    if (!fast) {
      bool ok = true;
#pragma unroll
      for (int t = 0; t < PF; ++t)
#pragma unroll
        for (int c = 0; c < kRowsNCB; ++c) ok &= t >= nb || fast_ok_bits<TT>(sval(t, c), bval(t, c));
      fast = rows_ballot(!ok) == 0;
    }
#pragma unroll
    for (int t = 0; t < PF; ++t)
      if (t < nb) {
        const unsigned char* xs = smem + (b0 + t) * 256;
        uint32_t st[kRowsNCB], bt[kRowsNCB];
#pragma unroll
        for (int c = 0; c < kRowsNCB; ++c) {
          st[c] = sval(t, c);
          bt[c] = bval(t, c);
        }
        if (fast)
          rows_step<TT, BITS, true, RBK>(wq[t], st, bt, xs, rstride, rows, acc);
        else
          rows_step<TT, BITS, false, RBK>(wq[t], st, bt, xs, rstride, rows, acc);
      }
  };
  for (int b0 = 0; b0 < S; b0 += PFMAX) {
    const int nb = min(PFMAX, S - b0);
    if constexpr (PFMAX >= 8) {
      if (nb > 4) {
        batch(b0, nb, std::integral_constant<int, 8>{});
        continue;
      }
    }
    if constexpr (PFMAX >= 4) {
      if (nb > 2) {
        batch(b0, nb, std::integral_constant<int, 4>{});
        continue;
      }
    }
    if (nb > 1) batch(b0, nb, std::integral_constant<int, 2>{});
    else batch(b0, nb, std::integral_constant<int, 1>{});
  }

  // 3. Store: element e of (row block rb, column block c) is row
  //    16 rb + 4 g + e, column n0 + 16 c + r.
#pragma unroll
  for (int c = 0; c < kRowsNCB; ++c) {
    const int col = n0 + 16 * c + r;
    if (col < n)
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * rb + 4 * g + e;
          if (row < m) y[(size_t)row * n + col] = TT::from_f32(acc[rb][c][e]);
        }
  }
}

size_t rows_lds(int m, int k) { return (size_t)m * (size_t)((k / 128 + 3) / 4) * 1024; }

template <typename TT, int BITS, int RBK, bool WIDE>
hipError_t launch_rows_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  const size_t lds = rows_lds(m, k);
  if (lds > 64 * 1024) {
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&qmm_rows_kernel<TT, BITS, RBK, WIDE>);
      hipFuncAttributes fa;
      hipError_t e = hipFuncGetAttributes(&fa, fn);
      if (e != hipSuccess) return e;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (attr != hipSuccess) return attr;
  }
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  hipLaunchKernelGGL((qmm_rows_kernel<TT, BITS, RBK, WIDE>), dim3((unsigned)((n + kRowsCols - 1) / kRowsCols)),
                     dim3(64 * kRowsWaves), lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), m, n, k, gs_shift);
  return hipGetLastError();
}

template <typename TT, int BITS, bool WIDE>
hipError_t launch_rows_w(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  if (m <= 16) return launch_rows_t<TT, BITS, 1, WIDE>(s, q, x, y, m, n, k);
  if (m <= 32) return launch_rows_t<TT, BITS, 2, WIDE>(s, q, x, y, m, n, k);
  if (m <= 48) return launch_rows_t<TT, BITS, 3, WIDE>(s, q, x, y, m, n, k);
  return launch_rows_t<TT, BITS, 4, WIDE>(s, q, x, y, m, n, k);
}

// Group size 64 with an even number of groups per row: the form with wide
// (scale, bias) loads.
template <typename TT, int BITS>
hipError_t launch_rows_b(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  if (q.gs == 64 && ((k / 64) & 1) == 0) return launch_rows_w<TT, BITS, true>(s, q, x, y, m, n, k);
  return launch_rows_w<TT, BITS, false>(s, q, x, y, m, n, k);
}

}  // namespace

bool qmm_rows_supported(const QuantArgs& q, int m, int n, int k) {
  if (q.bits != 4 && q.bits != 8) return false;
  if (q.dtype != CPQ_DTYPE_BF16 && q.dtype != CPQ_DTYPE_F16) return false;
  if (q.gs != 32 && q.gs != 64 && q.gs != 128) return false;
  if (m < 1 || m > 64 || n < 1 || k < 128 || k % 128 != 0) return false;
  if (rows_lds(m, k) > (size_t)kRowsXMax) return false;
  if ((uint64_t)n * (uint64_t)k * q.bits / 8 >= (1ull << 31) - (1ull << 20)) return false;
  if ((uint64_t)n * (uint64_t)(k / q.gs) * 2 >= (1ull << 31)) return false;
  return true;
}

int qmm_rows_workgroups(int n) { return (n + kRowsCols - 1) / kRowsCols; }

hipError_t launch_qmm_rows(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  if (!qmm_rows_supported(q, m, n, k)) return hipErrorInvalidValue;
  if (q.dtype == CPQ_DTYPE_BF16)
    return q.bits == 4 ? launch_rows_b<BF16, 4>(s, q, x, y, m, n, k) : launch_rows_b<BF16, 8>(s, q, x, y, m, n, k);
  return q.bits == 4 ? launch_rows_b<F16, 4>(s, q, x, y, m, n, k) : launch_rows_b<F16, 8>(s, q, x, y, m, n, k);
}

}  // namespace cpq
