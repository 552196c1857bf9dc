// Small-M quantized GEMM for gfx950: Y[M,N] = X[M,K] . dequant(W[N,K])^T for
// 1 <= M <= 64 activation rows, 4- and 8-bit weights, K a multiple of 256.
//
// Reference semantics: qmm_t_impl (kernels-mlx/mlx/backend/metal/kernels/
// quantized.h:1087-1213) -- each weight is dequantized to T as
// RNE_T(fmaf(scale, q, bias)), products accumulate in fp32, the output is
// rounded to T once.
//
// At a few dozen rows the weight stream (N*K*bits/8 bytes from HBM) is the
// work, every weight is dequantized exactly once, and a launch is short
// enough that its fixed latencies (kernel arguments, one memory round trip
// for the operands, the store) dominate: every load of a workgroup is issued
// before its first wait.  With MB 16-row blocks (M <= 16 * MB):
//   - workgroup = 512 threads = 8 waves, one tile of 16*MB columns of W;
//     wave w owns the 16 columns 16*(w % MB) of the tile and the K slice
//     w / MB (8/MB slices), i.e. every (8/MB)-th 256-element unit of the
//     workgroup's K range;
//   - the activation rows X[0..min(M, 16 MB)) of a K range of kb elements
//     (at most 128 KiB) are copied into LDS (buffer_load ... lds, 16-byte
//     units; unit c of row r is stored at position c ^ (r & 15), so the
//     operand reads below hit 16 distinct bank groups); a K range longer
//     than kb is walked in chunks;
//   - lane (column nl, group g) of a unit reads the 8 (4-bit) or 16 (8-bit)
//     words holding elements [64g, 64g+64) of the unit, 128 contiguous bytes
//     per column at 4-bit, and at k step s (0..7) dequantizes elements
//     64g+8s .. +7 into an MFMA B operand; the A operand of row r is the same
//     8 elements of X, read from LDS one step ahead.
//     v_mfma_f32_16x16x32_{bf16,f16}: A[m][k] in lane m + 16(k/8), B[k][n]
//     in lane n + 16(k/8), D[m][n] in lane n + 16(m/4), element m%4;
//   - the K slices are added through LDS in slice order; with M <= 16 one
//     workgroup covers all of K (no exchange between workgroups).  Past 16
//     rows the activation tile of a K range shrinks, so K is split over
//     `split` workgroups whose partial tiles are added, in part order, by the
//     last to finish (the exchange of the prefill kernel).
// Rows past M are never read or stored (an output row depends only on its
// own activation row); columns past N re-read column N-1 and are not stored.
#include <algorithm>
#include <type_traits>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int SKU = 256;           // k elements per unit (4 lane groups x 8 steps x 8)
constexpr int SUW = 2;             // most units of one wave per chunk
constexpr int SMAXSPLIT = 16;      // most K parts per tile
constexpr int SXMAX = 128 * 1024;  // most LDS bytes of the activation tile

// Split-K words in the scratch head (all zero between launches): per tile
// [t] the arrivals (low 8 bits) and, bit 8 + kk, part kk parked through its
// XCD's L2; the XCD each part runs on, plus one, [kSmallXcc + t*split + kk].
constexpr int kSmallMaxTiles = 4096;
constexpr int kSmallXcc = 10240;
constexpr int kSmallMaxParts = 6144;
constexpr size_t kSmall1Lds = 8 * 16384 + 7 * 64 * 16;  // per-wave activation pieces + parked K slices

template <typename TT, int BITS, int MB>
__global__ __launch_bounds__(512) void qmm_small_kernel(const uint32_t* __restrict__ w,
                                                        const uint16_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ biases,
                                                        const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                        int m, int n, int k, int gs_shift, int kb, int nch, int split,
                                                        int tiles, float* __restrict__ part,
                                                        unsigned int* __restrict__ counters, int xdma) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ uint32_t flags[2];
  constexpr int R = 16 * MB;      // activation rows of the tile
  constexpr int NB = 16 * MB;     // columns of the tile
  constexpr int NKS = 8 / MB;     // K slices
  constexpr int WPU = 2 * BITS;   // weight words of one lane per unit
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ct = wave % MB, ks = wave / MB;
  const int nl = lane & 15, g = lane >> 4;

  // Workgroup order: each XCD (linear ids congruent mod 8) takes a
  // contiguous run of (tile, part) pairs, part fastest, so the parts of a
  // tile normally share one L2.
  const int nwg = tiles * split;
  int v = blockIdx.x;
  if ((nwg & 7) == 0) v = (v & 7) * (nwg >> 3) + (v >> 3);
  const int kp = v % split, t = v / split;
  const int U = kb / SKU;   // units per chunk
  const int RU = kb / 8;    // 16-byte units per activation row
  const int G = k >> gs_shift;
  const int rows = min(m, R);

  const uint32_t xcc1 = (__builtin_amdgcn_s_getreg(20 | (31 << 11)) & 0xfu) + 1u;
  if (split > 1 && tid == 0)
    __hip_atomic_store(&counters[kSmallXcc + t * split + kp], xcc1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);
  const int col = t * NB + 16 * ct + nl;
  const bool col_ok = col < n;
  const int ccol = min(col, n - 1);
  const uint32_t* wrow = w + (size_t)ccol * ((size_t)k * BITS / 32);
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(scales + (size_t)ccol * G);
  const uint32_t* brow = reinterpret_cast<const uint32_t*>(biases + (size_t)ccol * G);
  const int nu = (U - ks + NKS - 1) / NKS;  // units of this wave per chunk
  const unsigned char* arow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) arow[mb] = smem + (size_t)(16 * mb + nl) * RU * 16;

  f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int ch = 0; ch < nch; ++ch) {
    const int k0 = (kp * nch + ch) * kb;
    if (ch > 0) __syncthreads();  // every wave done with the previous chunk's tile

    // 1. Activation rows into LDS: copy i (1 KiB) lands at byte 1024 i; lane
    //    l at position p = 64 i + l = row p / RU, stored unit p % RU, which
    //    holds unit (p % RU) ^ (row & 15) of the row's K range.  Copies whose
    //    first row is past M are skipped; a copy that starts inside M and
    //    runs past it re-reads row M-1.
    const int ncopies = R * RU / 64;
    constexpr int XPW = 16;  // most copies per wave (MB * kb / 256)
    u32x4 xv[XPW];
    if (xdma) {
      for (int i = wave; i < ncopies; i += 8) {
        if ((64 * i) / RU >= rows) break;
        const int p = 64 * i + lane;
        const int r = p / RU;
        const int c = (p - r * RU) ^ (r & 15);
        const int gr = min(r, m - 1);
        const uint32_t off = ((uint32_t)gr * (uint32_t)k + (uint32_t)k0 + (uint32_t)(8 * c)) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(smem + 1024 * i), 16,
                                                 off, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < XPW; ++j) {
        const int i = wave + 8 * j;
        if (i < ncopies && (64 * i) / RU < rows) {
          const int p = 64 * i + lane;
          const int r = p / RU;
          const int c = (p - r * RU) ^ (r & 15);
          const int gr = min(r, m - 1);
          const uint32_t off = ((uint32_t)gr * (uint32_t)k + (uint32_t)k0 + (uint32_t)(8 * c)) * 2u;
          xv[j] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0);
        }
      }
    }

    // 2. Weights and the scale / bias words of this lane's units (unit
    //    ks + NKS j), all issued before any wait; a unit past the chunk
    //    re-reads the last one and is not used.
    uint32_t wv[SUW][WPU];
    uint32_t sw[SUW], bw[SUW];
    int hs[SUW][2];
#pragma unroll
    for (int j = 0; j < SUW; ++j) {
      const int u = min(ks + NKS * j, U - 1);
      const int ku = k0 + SKU * u + 64 * g;  // first element of the lane's 64
      const uint32_t* p = wrow + (size_t)ku * BITS / 32;
#pragma unroll
      for (int q = 0; q < WPU / 4; ++q) {
        const u32x4 v4 = *reinterpret_cast<const u32x4*>(p + 4 * q);
        wv[j][4 * q] = v4.x;
        wv[j][4 * q + 1] = v4.y;
        wv[j][4 * q + 2] = v4.z;
        wv[j][4 * q + 3] = v4.w;
      }
      // Groups of elements ku .. ku+31 and ku+32 .. ku+63: both in the
      // 32-bit word of group pair (ku >> gs_shift) / 2.
      const int g0 = ku >> gs_shift, g1 = (ku + 32) >> gs_shift;
      sw[j] = srow[g0 >> 1];
      bw[j] = brow[g0 >> 1];
      hs[j][0] = g0 & 1;
      hs[j][1] = g1 & 1;
    }
    if (!xdma) {
#pragma unroll
      for (int j = 0; j < XPW; ++j) {
        const int i = wave + 8 * j;
        if (i < ncopies && (64 * i) / RU < rows) *reinterpret_cast<u32x4*>(smem + 1024 * i + 16 * lane) = xv[j];
      }
    }
    // The barrier waits for the LDS writes only: a unit's weights are
    // waited for where the unit starts, so the first units compute while
    // the later ones are still arriving (M = 64 at N = K = 4096: 13.1 ->
    // 12.5 us).  Copies into LDS count as loads, so they are waited for.
    if (xdma) wait_vmcnt<0>();
    lds_barrier();

    // 3. Dequantize and multiply; the next step's A operands are read while
    //    a step is dequantized.
#pragma unroll
    for (int j = 0; j < SUW; ++j) {
      if (j < nu) {
        const int u = ks + NKS * j;
        float sf[2], bf[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t sh = hs[j][h] ? sw[j] >> 16 : sw[j] & 0xffffu;
          const uint32_t bh = hs[j][h] ? bw[j] >> 16 : bw[j] & 0xffffu;
          sf[h] = TT::to_f32((uint16_t)sh);
          bf[h] = TT::to_f32((uint16_t)bh);
        }
        const int cu = 32 * u + 8 * g;
        u32x4 a[2][MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) a[0][mb] = *reinterpret_cast<const u32x4*>(arow[mb] + ((cu ^ nl) << 4));
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if (s < 7)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              a[(s + 1) & 1][mb] = *reinterpret_cast<const u32x4*>(arow[mb] + (((cu + s + 1) ^ nl) << 4));
          const int h = s >> 2;
          uint32_t bo[4];
          dequant8<TT, BITS, 0>(&wv[j][BITS == 4 ? s : 2 * s], sf[h], sf[h] * 0.0625f, bf[h], bo);
          const u32x4 bop = {bo[0], bo[1], bo[2], bo[3]};
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[mb] = Mfma16<TT>::run(a[s & 1][mb], bop, acc[mb]);
        }
      }
    }
  }

  // 4. The K slices of each column tile, in slice order: slices 1.. park
  //    their tiles after the activation tile, slice 0 adds them.
  float* red = reinterpret_cast<float*>(smem + (size_t)R * RU * 16);
  if (NKS > 1) {
    if (ks > 0)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        *reinterpret_cast<f32x4*>(red + ((((ks - 1) * MB + ct) * MB + mb) * 64 + lane) * 4) = acc[mb];
    __syncthreads();
    if (ks == 0)
#pragma unroll
      for (int kk = 1; kk < NKS; ++kk)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[mb] = acc[mb] + *reinterpret_cast<const f32x4*>(red + ((((kk - 1) * MB + ct) * MB + mb) * 64 + lane) * 4);
  }

  // 5. Split K: the prefill kernel's exchange.  A workgroup parks its partial
  //    tile, waits until every store is complete and only then counts its
  //    arrival, adding bit 8 + kp when it parked through its L2; the last
  //    arriver (count split - 1) thus finds every other part complete and
  //    adds the parts in part order.  Parts of workgroups that found every
  //    part of the tile on their XCD go through its L2 (plain stores and
  //    loads), others with the sc1 policy (written through to, and read
  //    from, the memory side, as agent-scope atomics are).  Lane kk of
  //    wave 0 reads part kk's XCD word.
  if (split > 1) {
    constexpr int SC1 = 16;
    if (wave == 0) {
      uint32_t xw = xcc1;
      if (lane < split && lane != kp)
        xw = __hip_atomic_load(&counters[kSmallXcc + t * split + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool all_here = __ballot(xw != xcc1) == 0ull;
      if (lane == 0) flags[1] = all_here ? 1u : 0u;
    }
    __syncthreads();
    const bool local = flags[1] != 0u;
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(part + (size_t)t * split * MB * MB * 256), 0, (int)(split * MB * MB * 1024), 0x00020000);
    auto off = [&](int kk, int mb) { return (uint32_t)((((kk * MB + ct) * MB + mb) * 64 + lane) * 16); };
    if (ks == 0)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const u32x4 v4 = __builtin_bit_cast(u32x4, acc[mb]);
        if (local)
          __builtin_amdgcn_raw_buffer_store_b128(v4, pr, off(kp, mb), 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b128(v4, pr, off(kp, mb), 0, SC1);
      }
    __builtin_amdgcn_s_waitcnt(0);  // every store of this thread complete
    __syncthreads();
    if (tid == 0)
      flags[0] = __hip_atomic_fetch_add(&counters[t], 1u + (local ? (256u << kp) : 0u), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if ((flags[0] & 255u) != (unsigned int)(split - 1)) return;
    // Parts parked through the L2: a part parks there only when all parts,
    // this one included, run on its XCD.
    const uint32_t l2_parts = flags[0] >> 8;
    const uint32_t others = ((1u << split) - 1u) & ~(1u << kp);
    if (ks == 0) {
      f32x4 sum[MB];
      if (l2_parts == others) {
        // Every part through this L2: four parts' loads in flight at a time.
        for (int k4 = 0; k4 < split; k4 += 4) {
          f32x4 pv[4][MB];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k4 + i < split)
#pragma unroll
              for (int mb = 0; mb < MB; ++mb)
                pv[i][mb] = k4 + i == kp
                                ? acc[mb]
                                : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off(k4 + i, mb), 0, 0));
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (k4 + i < split)
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) sum[mb] = k4 + i == 0 ? pv[i][mb] : sum[mb] + pv[i][mb];
        }
      } else {
        for (int kk = 0; kk < split; ++kk) {
          f32x4 pv[MB];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if (kk == kp)
              pv[mb] = acc[mb];
            else if ((l2_parts >> kk) & 1u)
              pv[mb] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off(kk, mb), 0, 0));
            else
              pv[mb] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off(kk, mb), 0, SC1));
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) sum[mb] = kk == 0 ? pv[mb] : sum[mb] + pv[mb];
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = sum[mb];
    }
    if (wave == 0) {
      if (lane == 0) __hip_atomic_store(&counters[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane < split)
        __hip_atomic_store(&counters[kSmallXcc + t * split + lane], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // 6. Store: element i of row block mb is row 16 mb + 4g + i, column col.
  if (ks == 0 && col_ok) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * g + i;
        if (row < m) y[(size_t)row * n + col] = TT::from_f32(acc[mb][i]);
      }
  }
}

// Up to 16 rows: one workgroup per 16 columns over all of K.  Wave w owns
// the 256-element units w, w+8, w+16, ... of K, two per batch, and stages the
// activation slices of its own units in a private 16 KiB of LDS, so waves
// never wait for each other until their K slices are added (through LDS, in
// slice order).
//   - Weights: load q of a unit reads, for lane (column nl, group g), the 16
//     bytes at 64q + 16g of the column's bytes of the unit (one 64-byte
//     segment per column per instruction), i.e. words 16q + 4g + i.  Step s
//     (0..7) consumes word s of the lane's list at 4-bit and words 2s, 2s+1
//     at 8-bit.
//   - Activations: one 1 KiB load per row per batch (lanes 0..31 the 32
//     16-byte pieces of the batch's first unit, lanes 32..63 of its second),
//     piece P of row r stored at position P ^ r; rows past M are not read
//     (their A rows only feed output rows that are never stored).
//   - At step s the A operand of lane (row nl, group g) is the piece holding
//     the 8 elements of the lane's weight word(s) s, read from LDS; the pieces
//     that 16 rows read at one step sit at 16 distinct positions.
// Every global access is a buffer load at a per-lane base plus a fixed or
// scalar offset.
template <int BITS>
__device__ __forceinline__ int small1_piece(int g, int s) {
  if constexpr (BITS == 4) return 16 * (s >> 2) + 4 * g + (s & 3);
  else return 8 * (s >> 1) + 2 * g + (s & 1);
}

template <typename TT, int BITS>
__global__ __launch_bounds__(512) void qmm_small1_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                         int m, int n, int k, int gs_shift) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int WPU = 2 * BITS;               // weight words of one lane per unit
  constexpr int UB = 2;                       // units per batch
  constexpr int RUNS = BITS == 4 ? 2 : 4;     // runs of one group per lane per unit
  constexpr int RUNLEN = BITS == 4 ? 32 : 16; // elements per run
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int col = blockIdx.x * 16 + nl;
  const int ccol = min(col, n - 1);
  const int G = k >> gs_shift;
  const int nu = (k / SKU - wave + 7) >> 3;  // units w + 8j of this wave
  const int rows = min(m, 16);
  const uint32_t rowbytes = (uint32_t)k * BITS / 8u;
  unsigned char* xs = smem + wave * 16384;                 // [16 rows][64 pieces of 16 B]
  f32x4* red = reinterpret_cast<f32x4*>(smem + 8 * 16384);  // [7][64]
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)scales, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc((void*)biases, 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);
  // Unit j of this wave starts at element SKU * (wave + 8j).
  const uint32_t wbase = (uint32_t)ccol * rowbytes + (uint32_t)(SKU * wave) * BITS / 8u + 16u * g;
  const uint32_t wstep = 8u * SKU * BITS / 8u;  // bytes between a lane's units
  const uint32_t cbase = (uint32_t)ccol * (uint32_t)G;
  const uint32_t xbase = ((uint32_t)(SKU * wave + 8 * SKU * (lane >> 5)) + 8u * (lane & 31)) * 2u;
  const uint32_t xrowb = (uint32_t)k * 2u;

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int jb = 0; jb < nu; jb += UB) {
    // 1. Loads (a unit past the wave's range re-reads its last and is not used).
    uint32_t wv[UB][WPU], sw[UB][RUNS], bw[UB][RUNS];
    int hs[UB][RUNS];
#pragma unroll
    for (int jj = 0; jj < UB; ++jj) {
      const int j = min(jb + jj, nu - 1);
#pragma unroll
      for (int q = 0; q < WPU / 4; ++q) {
        const u32x4 v = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wbase + 64u * q, (int)(j * wstep), 0));
        wv[jj][4 * q] = v.x;
        wv[jj][4 * q + 1] = v.y;
        wv[jj][4 * q + 2] = v.z;
        wv[jj][4 * q + 3] = v.w;
      }
    }
#pragma unroll
    for (int jj = 0; jj < UB; ++jj) {
      const int j = min(jb + jj, nu - 1);
      const int eu = SKU * (wave + 8 * j);
#pragma unroll
      for (int h = 0; h < RUNS; ++h) {
        // Run h: the elements of load h -- 4-bit: words 16h + 4g .. +3,
        // elements [128h + 32g, +32); 8-bit: elements [64h + 16g, +16).
        const int grp = (eu + (BITS == 4 ? 128 * h + 32 * g : 64 * h + 16 * g)) >> gs_shift;
        const uint32_t off = (cbase + (uint32_t)(grp & ~1)) * 2u;
        sw[jj][h] = __builtin_amdgcn_raw_buffer_load_b32(sr, off, 0, 0);
        bw[jj][h] = __builtin_amdgcn_raw_buffer_load_b32(br, off, 0, 0);
        hs[jj][h] = grp & 1;
      }
    }
    u32x4 xv[16];
    const int xsoff = jb * 8 * SKU * 2;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (r < rows)
        xv[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xbase + xrowb * r, xsoff, 0));

    // 2. Activation pieces into this wave's LDS, after every read of the
    //    previous batch.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (r < rows) *reinterpret_cast<u32x4*>(xs + r * 1024 + ((lane ^ r) << 4)) = xv[r];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 3. Dequantize and multiply.
    const unsigned char* arow = xs + nl * 1024;
#pragma unroll
    for (int jj = 0; jj < UB; ++jj) {
      if (jb + jj < nu) {
        float sf[RUNS], bf[RUNS];
#pragma unroll
        for (int h = 0; h < RUNS; ++h) {
          sf[h] = TT::to_f32((uint16_t)(hs[jj][h] ? sw[jj][h] >> 16 : sw[jj][h] & 0xffffu));
          bf[h] = TT::to_f32((uint16_t)(hs[jj][h] ? bw[jj][h] >> 16 : bw[jj][h] & 0xffffu));
        }
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          const int h = BITS == 4 ? st >> 2 : st >> 1;
          const int piece = 32 * jj + small1_piece<BITS>(g, st);
          const u32x4 a = *reinterpret_cast<const u32x4*>(arow + ((piece ^ nl) << 4));
          uint32_t bo[4];
          dequant8<TT, BITS, 0>(&wv[jj][BITS == 4 ? st : 2 * st], sf[h], sf[h] * 0.0625f, bf[h], bo);
          acc = Mfma16<TT>::run(a, u32x4{bo[0], bo[1], bo[2], bo[3]}, acc);
        }
      }
    }
  }

  // 4. K slices in order: slices 1..7 park, slice 0 adds and stores (element
  //    i of lane (nl, g) is row 4g + i, column col).
  if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 7; ++i) acc = acc + red[i * 64 + lane];
    if (col < n)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 4 * g + i;
        if (row < m) y[(size_t)row * n + col] = TT::from_f32(acc[i]);
      }
  }
}

// Raises one instantiation's dynamic-LDS limit to what the CU leaves beside
// its static LDS, once per process.
template <typename TT, int BITS, int MB>
hipError_t small_allow_lds() {
  static const hipError_t e = [] {
    const void* fn = reinterpret_cast<const void*>(&qmm_small_kernel<TT, BITS, MB>);
    hipFuncAttributes fa;
    hipError_t r = hipFuncGetAttributes(&fa, fn);
    if (r != hipSuccess) return r;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(160 * 1024 - fa.sharedSizeBytes));
  }();
  return e;
}

int small_mb(int m) { return m <= 16 ? 1 : m <= 32 ? 2 : 4; }

// Largest K chunk: the activation tile within 128 KiB and at most SUW units
// per wave.
int small_kb_max(int mb) { return std::min(SXMAX / (32 * mb), SUW * SKU * (8 / mb)); }

// Activation tile plus the K-slice tiles parked for the slice sum.
size_t small_lds(int mb, int kb) { return (size_t)32 * mb * kb + (size_t)(8 / mb - 1) * mb * mb * 1024; }

// Split-K scratch: arrival words, then one partial tile (MB*MB KiB) per part.
size_t small_scratch(long tiles, int split, int mb) {
  return split > 1 ? kWideCounterBytes + (size_t)tiles * split * mb * mb * 1024 : 0;
}

}  // namespace

SmallPlan qmm_small_plan(const QuantArgs& q, int m, int n, int k, int cu_count, size_t scratch_cap) {
  SmallPlan p{0, 0, 0, 0, 0};
  if ((q.bits != 4 && q.bits != 8) || (q.dtype != CPQ_DTYPE_BF16 && q.dtype != CPQ_DTYPE_F16)) return p;
  if ((q.gs != 32 && q.gs != 64 && q.gs != 128) || m < 1 || m > 64 || n < 1 || k < SKU || k % SKU != 0) return p;
  if ((uint64_t)m * (uint64_t)k * 2u >= (1ull << 31)) return p;
  const int mb = small_mb(m), kbmax = small_kb_max(mb);
  if (mb == 1) {
    // Up to 16 rows: all of K per workgroup, operands in registers.
    if ((uint64_t)n * (uint64_t)k * (uint64_t)q.bits / 8u >= (1ull << 31)) return p;
    p.split = 1;
    p.nch = 1;
    p.kb = k;
    p.mb = 1;
    return p;
  }
  const long tiles = (n + 16 * mb - 1) / (16 * mb);
  const long cus = cu_count > 0 ? cu_count : 256;
  const int ku = k / SKU;
  // CPQ_SMALL_SPLIT / CPQ_SMALL_NCH force the K split and the chunks per
  // workgroup (tuning hooks, read once per process).
  static const int f_split = env_int("CPQ_SMALL_SPLIT", 0), f_nch = env_int("CPQ_SMALL_NCH", 0);
  // Chunks of a K range of ku/d units: the fewest with a chunk <= kbmax.
  auto chunks = [&](int d) {
    const int kud = ku / d;
    for (int c = 1; c <= kud; ++c)
      if (kud % c == 0 && (k / d / c) <= kbmax && (f_nch == 0 || c == f_nch)) return c;
    return 0;
  };
  // Up to 16 rows one workgroup covers all of K (no exchange); past that,
  // the fewest K parts that give every CU a workgroup, or the most allowed.
  int best = 0, best_c = 0;
  for (int d = 1; d <= std::min(ku, SMAXSPLIT); ++d) {
    if (ku % d != 0 || (f_split && d != f_split)) continue;
    const int c = chunks(d);
    if (c == 0) continue;
    if (d > 1 && (tiles > kSmallMaxTiles || tiles * d > kSmallMaxParts || small_scratch(tiles, d, mb) > scratch_cap))
      continue;
    best = d;
    best_c = c;
    if (mb == 1 || tiles * d >= cus) break;
  }
  if (best == 0) return p;
  p.split = best;
  p.nch = best_c;
  p.kb = k / best / best_c;
  p.mb = mb;
  p.scratch_bytes = small_scratch(tiles, best, mb);
  return p;
}

hipError_t launch_qmm_small(hipStream_t s, const SmallPlan& p, void* scratch, const QuantArgs& q, const void* x,
                            void* y, int m, int n, int k) {
  if (p.split < 1 || (p.split > 1 && !scratch)) return hipErrorInvalidValue;
  const int tiles = (n + 16 * p.mb - 1) / (16 * p.mb);
  const int gs_shift = q.gs == 32 ? 5 : q.gs == 64 ? 6 : 7;
  unsigned int* counters = static_cast<unsigned int*>(scratch);
  float* part = scratch ? reinterpret_cast<float*>(static_cast<char*>(scratch) + kWideCounterBytes) : nullptr;
  if (p.mb == 1) {
    auto go1 = [&](auto kern) -> hipError_t {
      static const hipError_t a = [&] {
        hipFuncAttributes fa;
        hipError_t r = hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(kern));
        if (r != hipSuccess) return r;
        return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)(160 * 1024 - fa.sharedSizeBytes));
      }();
      if (a != hipSuccess) return a;
      hipLaunchKernelGGL(kern, dim3((unsigned)((n + 15) / 16)), dim3(512), kSmall1Lds, s, q.w,
                         static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                         static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), m, n, k, gs_shift);
      return hipGetLastError();
    };
    if (q.dtype == CPQ_DTYPE_BF16) return q.bits == 4 ? go1(qmm_small1_kernel<BF16, 4>) : go1(qmm_small1_kernel<BF16, 8>);
    if (q.dtype == CPQ_DTYPE_F16) return q.bits == 4 ? go1(qmm_small1_kernel<F16, 4>) : go1(qmm_small1_kernel<F16, 8>);
    return hipErrorInvalidValue;
  }
  const size_t lds = small_lds(p.mb, p.kb);
  // CPQ_SMALL_XDMA=1 stages the activation rows with buffer_load ... lds
  // instead of through registers (tuning hook, read once per process).
  static const int xdma = env_int("CPQ_SMALL_XDMA", 0);
  auto go = [&](auto tt, auto bits, auto mbc) -> hipError_t {
    using TT = decltype(tt);
    constexpr int B = decltype(bits)::value, MB = decltype(mbc)::value;
    if (lds > (size_t)64 * 1024) {
      const hipError_t a = small_allow_lds<TT, B, MB>();
      if (a != hipSuccess) return a;
    }
    hipLaunchKernelGGL((qmm_small_kernel<TT, B, MB>), dim3((unsigned)(tiles * p.split)), dim3(512), lds, s, q.w,
                       static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), m, n, k, gs_shift, p.kb, p.nch,
                       p.split, tiles, part, counters, xdma);
    return hipGetLastError();
  };
  using M1 = std::integral_constant<int, 1>;
  using M2 = std::integral_constant<int, 2>;
  using M4 = std::integral_constant<int, 4>;
  auto by_mb = [&](auto tt, auto bits) -> hipError_t {
    if (p.mb == 1) return go(tt, bits, M1{});
    if (p.mb == 2) return go(tt, bits, M2{});
    return go(tt, bits, M4{});
  };
  using B4 = std::integral_constant<int, 4>;
  using B8 = std::integral_constant<int, 8>;
  if (q.dtype == CPQ_DTYPE_BF16) return q.bits == 4 ? by_mb(BF16{}, B4{}) : by_mb(BF16{}, B8{});
  if (q.dtype == CPQ_DTYPE_F16) return q.bits == 4 ? by_mb(F16{}, B4{}) : by_mb(F16{}, B8{});
  return hipErrorInvalidValue;
}

}  // namespace cpq
