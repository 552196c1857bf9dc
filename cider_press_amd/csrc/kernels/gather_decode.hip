// Routed experts at decode shapes: a few (token, expert) rows, each against
// its own expert's weight matrix.
//
// Reference op: the rhs-indexed gather of MLX, affine_gather_qmv_fast /
// affine_gather_qmv (kernels-mlx/mlx/backend/metal/kernels/quantized.h:
// 1905-2028), which runs one GEMV per (row, expert).  Numerics as every path
// here: each weight is dequantized to T (RNE of fmaf(s, q, b)), products
// accumulate in fp32 on the matrix cores, the output is rounded to T once.
//
// HBM-bound.  Rows that pick the same expert share one pass over its
// weights, so the bytes read are those of the distinct experts touched.
//   - Workgroup (column block cb, slot u): 16 output columns of the u-th
//     distinct expert of the call (distinct experts numbered by the first row
//     that names them).  Every wave reads all of rhs (n_rows <= 64: one load
//     per lane) and derives the slot's expert and its rows with ballots, so no
//     sort or pre-pass kernel runs; slots past the number of distinct experts
//     exit at once, except the first of them, which zeroes this column block
//     of rows whose expert index is out of range.
//   - The slot's rows go through the matrix cores kDecPass at a time (a
//     slot at decode holds one or two rows; a small pass keeps the LDS per
//     workgroup small, so several workgroups share a CU): MFMA
//     16x16x32 with A = the rows' activations (staged in LDS) and B = 8
//     dequantized weights per lane, lane (r, g) holding column n0 + r and
//     chunk 4j + g of step j (128 k per step), as in the decode kernel.
//   - The 4 waves of a workgroup split K into KW contiguous step ranges and
//     the columns into 4 / KW blocks of 16 (KW chosen by the grid size, see
//     gather_decode_kw); each wave issues the weight
//     and (scale, bias) loads of its range (up to 8 steps) before staging its
//     own activation slices, votes on the single-FMA dequantization within
//     the wave, then multiplies.  The K parts are summed through LDS in wave
//     order.
//   - Index checks: rows with an out-of-range expert or activation index are
//     written as zeros and counted into *status (by workgroup (0, 0)),
//     together with descents of a routing declared sorted; no index is used
//     to address memory before it is checked.
#include <algorithm>
#include <type_traits>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int kDecPF = 8;       // steps of loads in flight per wave
constexpr int kDecMaxRows = 64; // rows of one call (one lane each)
constexpr int kDecPass = 4;     // rows of a slot per pass (decode slots hold one or two)
constexpr int kDensePass = 8;   // rows per pass (workgroup) of the dense small-M form
constexpr int kDecWaves = 4;    // waves per workgroup: KW split K, 4 / KW column blocks

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

template <int BITS>
__device__ __forceinline__ void dec_load(__amdgpu_buffer_rsrc_t wr, uint32_t voff, uint32_t* dst) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff, 0, 0));
  dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
  if constexpr (BITS == 8) {
    const u32x4 v1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff + 16, 0, 0));
    dst[4] = v1.x; dst[5] = v1.y; dst[6] = v1.z; dst[7] = v1.w;
  }
}

// Four MFMAs of one step: activation slices from the wave's LDS rows, the
// lane's chunk dequantized slice by slice.
template <typename TT, int BITS, bool FAST>
__device__ __forceinline__ f32x4 dec_step(const uint32_t* wq, uint32_t sv, uint32_t bv, const unsigned char* xrow,
                                          int m, f32x4 acc) {
  const float s = TT::to_f32((uint16_t)sv), b = TT::to_f32((uint16_t)bv);
  const float s16 = s * 0.0625f, c0 = fmaf(-1024.f, s, b), c1 = fmaf(-64.f, s, b);
  const int g4 = (threadIdx.x >> 4) & 3;
  const int km = swz_key(m);
  const u32x4 a0 = *reinterpret_cast<const u32x4*>(xrow + (((4 * g4 + 0) ^ km) << 4));
  const u32x4 a1 = *reinterpret_cast<const u32x4*>(xrow + (((4 * g4 + 1) ^ km) << 4));
  const u32x4 a2 = *reinterpret_cast<const u32x4*>(xrow + (((4 * g4 + 2) ^ km) << 4));
  const u32x4 a3 = *reinterpret_cast<const u32x4*>(xrow + (((4 * g4 + 3) ^ km) << 4));
  acc = Mfma16<TT>::run(a0, dequant_slice<TT, BITS, FAST, 0>(wq, s, s16, b, c0, c1), acc);
  acc = Mfma16<TT>::run(a1, dequant_slice<TT, BITS, FAST, 1>(wq, s, s16, b, c0, c1), acc);
  acc = Mfma16<TT>::run(a2, dequant_slice<TT, BITS, FAST, 2>(wq, s, s16, b, c0, c1), acc);
  acc = Mfma16<TT>::run(a3, dequant_slice<TT, BITS, FAST, 3>(wq, s, s16, b, c0, c1), acc);
  return acc;
}

// DENSE: the same kernel as a small-M matmul (one weight matrix, rows
// 0..n_rows-1 of x and y; lhs, rhs and status unused): slot u is then the
// u-th pass of rows_max rows.
template <typename TT, int BITS, int KW, bool DENSE, bool WIDE>
__global__ __launch_bounds__(64 * kDecWaves) __attribute__((amdgpu_waves_per_eu(BITS == 4 ? 4 : 3))) void gather_decode_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ x, int x_rows, const uint32_t* __restrict__ lhs, const uint32_t* __restrict__ rhs,
    int n_rows, uint16_t* __restrict__ y, int n_experts, int n, int k, int gs_shift, int sorted, int rows_max,
    int steps_w, unsigned int* __restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int CB = kDecWaves / KW;  // 16-column blocks per workgroup
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kw = wave % KW, cbl = wave / KW;
  const int nw0 = blockIdx.x * 16 * CB;  // first column of the workgroup
  const int n0 = nw0 + 16 * cbl;         // first column of this wave's block
  const int u = blockIdx.y;

  uint32_t eu = 0, xr = 0;
  uint64_t rows = 0, lvmask = ~0ull;
  int nr = 0, rowbase = 0;
  if constexpr (DENSE) {
    rowbase = u * rows_max;
    nr = min(rows_max, n_rows - rowbase);
  } else {
    // 1. Routing: lane i holds row i's expert and activation row.
    const bool in = lane < n_rows;
    const uint32_t e = in ? rhs[lane] : 0xffffffffu;
    xr = in ? (lhs ? lhs[lane] : (uint32_t)lane) : 0u;
    const bool ev = in && e < (uint32_t)n_experts;
    const bool lv = in && xr < (uint32_t)x_rows;
    const uint64_t valid = ballot(ev);
    lvmask = ballot(lv);  // rows whose activation index is in range
    uint64_t later = 0;   // rows naming an expert an earlier row already named
    for (int j = 0; j < n_rows; ++j) {
      const uint32_t ej = __builtin_amdgcn_readlane(e, j);
      const uint64_t same = ballot(ev && e == ej);
      later |= same & (~0ull << j << 1);
    }
    const uint64_t first = valid & ~later;
    const int nuniq = __builtin_popcountll(first);
    if (blockIdx.x == 0 && u == 0) {
      const uint32_t nxt = (in && lane + 1 < n_rows) ? rhs[lane + 1] : 0xffffffffu;
      const int bad = __builtin_popcountll(ballot(in && (!ev || !lv))) +
                      (sorted ? __builtin_popcountll(ballot(lane + 1 < n_rows && e > nxt)) : 0);
      if (wave == 0 && lane == 0 && bad) atomicAdd(status, (unsigned)bad);
    }
    if (u >= nuniq) {
      if (u == nuniq) {  // zero this column block of rows with an out-of-range expert
        const uint64_t badrows = ballot(in && !ev);
        for (int t = threadIdx.x; t < 64 * 16 * CB; t += 64 * kDecWaves) {
          const int r = t / (16 * CB), c = nw0 + t % (16 * CB);
          if (((badrows >> r) & 1) && c < n) y[(size_t)r * n + c] = 0;
        }
      }
      return;
    }
    uint64_t fm = first;
    for (int i = 0; i < u; ++i) fm &= fm - 1;
    const int lead = __builtin_ctzll(fm);
    eu = __builtin_amdgcn_readlane(e, lead);
    rows = ballot(ev && e == eu);
    nr = __builtin_popcountll(rows);
  }

  // 2. This wave's K range and weight stream of expert eu.
  const int G = k >> gs_shift;
  const int S = (k + 127) >> 7;  // steps of 128 (the last one partial when K % 128 != 0)
  // Wave kw takes steps [kw SW, (kw + 1) SW) of S, SW = ceil(S / KW): with
  // KW = 4 (or 1), a K zero-padded to the next multiple of 512 keeps every
  // wave's steps and adds only zero steps.
  const int SW = (S + KW - 1) / KW;
  const int js = min(kw * SW, S), je = min(js + SW, S);
  const int nst = je - js;
  const int r = lane & 15, g = lane >> 4;
  const uint32_t rowbytes = (uint32_t)k * BITS / 8u;
  const size_t ewords = (size_t)n * (size_t)k * BITS / 32;
  const size_t egroups = (size_t)n * (size_t)G;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (size_t)eu * ewords), 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(scales + (size_t)eu * egroups), 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(biases + (size_t)eu * egroups), 0, (int)((uint32_t)n * (uint32_t)G * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xs =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)x_rows * (uint32_t)k * 2u), 0x00020000);
  // Columns past N read zeros through the range check (offsets past 2^31,
  // beyond every range; never stored).
  const bool col_ok = n0 + r < n;
  const uint32_t voff0 =
      col_ok ? (uint32_t)(n0 + r) * rowbytes + (uint32_t)(4 * js + g) * (BITS * 4u) : 0x80000000u;
  const uint32_t coff0 = col_ok ? (uint32_t)(n0 + r) * (uint32_t)G : 0x40000000u;

  const int RB = min(steps_w, kDecPF) * 256;  // bytes of one activation row in the wave's region
  unsigned char* xw = smem + (size_t)wave * rows_max * RB;
  float* red = reinterpret_cast<float*>(smem + (size_t)kDecWaves * rows_max * RB);  // [waves][64][4]
  int* rlist = reinterpret_cast<int*>(red + kDecWaves * 256);                           // [64]

  // The slot's rows in order: rank -> row.
  if constexpr (DENSE) {
    if (lane < nr) rlist[lane] = rowbase + lane;
  } else {
    if ((rows >> lane) & 1) rlist[__builtin_popcountll(rows & ((1ull << lane) - 1))] = lane;
  }
  __syncthreads();

  for (int p0 = 0; p0 < nr; p0 += rows_max) {
    const int np = min(rows_max, nr - p0);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    // Steps per batch: 8 for one row, 4 for up to 4 rows, else 2; the
    // pass's activation pieces of a batch (16 per row and step) then fit the
    // XP slots per lane of the batch form that runs it (see batch below).
    const int bmax = np == 1 ? 8 : np <= 4 ? 4 : 2;
    // One batch of nb <= PF steps.  2a. The pass's activation slices (row m,
    // step t, 16-byte piece p in natural order, stored at slot p ^ swz_key(m) of the
    // row's step) are requested first: their addresses are known from the
    // routing loads already (a row's activation index comes from the routing
    // lane holding it by a lane shuffle).  2b. Then (scale, bias) of each
    // step, then the weights: the vote needs only the former, and step t's
    // multiply waits for its own weights alone.  Every load is issued in one
    // straight run, the PF slots past nb at an offset past every range (they
    // read zeros): loads under a branch would make the compiler wait for each
    // step's data before issuing the next.
    auto batch = [&](int b0, int nb, auto pfc) {
      constexpr int PF = decltype(pfc)::value;
      // PF 8 runs one row (<= 128 pieces), PF 4 up to 4 rows and PF 2 up to
      // 8 (<= 256), PF 1 up to 8 (<= 128).
      constexpr int XP = (PF == 8 || PF == 1) ? 2 : 4;
      const int pieces = np * nb * 16;
      // q / (16 nb) as (q * inv) >> 16: exact for every q < 783 at these
      // divisors (q < 256 here), two VALU instead of a division.
      const uint32_t inv = (65536u + 16u * nb - 1u) / (16u * nb);
      u32x4 xv[XP];
      int xdst[XP];
#pragma unroll
      for (int i = 0; i < XP; ++i) {
        xdst[i] = -1;
        if (i == 0 || 64 * i < pieces) {  // uniform
          const int q = lane + 64 * i;
          const int qc = q < pieces ? q : 0;
          const int m = (int)(((uint32_t)qc * inv) >> 16), rem = qc - m * (nb * 16), t = rem >> 4, pc = rem & 15;
          const int row = rlist[p0 + m];
          const uint32_t xrow = lhs ? (uint32_t)__shfl((int)xr, row, 64) : (uint32_t)row;
          xdst[i] = q < pieces ? m * RB + t * 256 + ((pc ^ swz_key(m)) << 4) : -1;
          const uint32_t kk = (uint32_t)(js + b0 + t) * 128u + (uint32_t)pc * 8u;  // first element of the piece
          const uint32_t off =
              q < pieces && xrow < (uint32_t)x_rows && kk < (uint32_t)k ? (xrow * (uint32_t)k + kk) * 2u : 0x80000000u;
          xv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xs, off, 0, 0));
        }
      }
      uint32_t wq[PF][BITS];
      // (scale, bias) of each step.  WIDE (group size 64, an even number of
      // groups per row, so K is a multiple of 128 and every step of the
      // batch is whole): the column's words for the batch's steps in one or
      // two wide loads (word T holds step T's two groups; a 2-byte load per
      // step and value cost the 4-token up projection 3.3 us), then the
      // lane's halves of steps t, t + 1 packed into one register (the
      // packed form the vote reads), 16 bits per step.  Otherwise a 16-bit
      // load per step and value; chunks past K (a partial last step) read
      // zeros like the slots past the batch.
      constexpr int NP = WIDE ? (PF + 1) / 2 : PF;
      uint32_t sv[NP], bv[NP];
      bool live[PF];
#pragma unroll
      for (int t = 0; t < PF; ++t) {
        const uint32_t ck = (uint32_t)(4 * (js + b0 + t) + g) * 32u;
        live[t] = t < nb && ck < (uint32_t)k;
      }
      if constexpr (WIDE) {
        uint32_t sw[PF], bw[PF];
        const uint32_t wo = (coff0 + 2u * (uint32_t)(js + b0)) * 2u;  // past 2^31 for columns past N
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
          sv[j] = __builtin_amdgcn_perm(sw[t1], sw[2 * j], psel);
          bv[j] = __builtin_amdgcn_perm(bw[t1], bw[2 * j], psel);
        }
      } else {
#pragma unroll
        for (int t = 0; t < PF; ++t) {
          const uint32_t ck = (uint32_t)(4 * (js + b0 + t) + g) * 32u;
          const uint32_t gi = coff0 + (ck >> gs_shift);
          const uint32_t so = live[t] ? gi * 2u : 0x80000000u;
          sv[t] = __builtin_amdgcn_raw_buffer_load_b16(sr, so, 0, 0);
          bv[t] = __builtin_amdgcn_raw_buffer_load_b16(br, so, 0, 0);
        }
      }
      // Step t's 16-bit scale / bias (bits 0..15 of the result).
      auto sval = [&](int t) -> uint32_t {
        if constexpr (WIDE) return (t & 1) ? sv[t >> 1] >> 16 : sv[t >> 1];
        else return sv[t];
      };
      auto bval = [&](int t) -> uint32_t {
        if constexpr (WIDE) return (t & 1) ? bv[t >> 1] >> 16 : bv[t >> 1];
        else return bv[t];
      };
#pragma unroll
      for (int t = 0; t < PF; ++t)
        dec_load<BITS>(wr, live[t] ? voff0 + (uint32_t)(b0 + t) * (16u * BITS) : 0x80000000u, wq[t]);
#pragma unroll
      for (int i = 0; i < XP; ++i)
        if (xdst[i] >= 0) *reinterpret_cast<u32x4*>(xw + xdst[i]) = interleave_x<BITS>(xv[i]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();  // the staged slices before any lane reads them
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // 2c. Vote (within the wave) on the single-FMA dequantization: the
      //     packed exponent check over the batch's (scale, bias) pairs, two
      //     per word (slots past the batch or past K count as (1, 1), which
      //     passes), and the exact per-group check only when some lane
      //     fails it.
      constexpr uint32_t kOne = Sig16<TT>::bf16 ? 0x3F80u : 0x3C00u;
      FastQuick fq;
      fast_quick_init(fq);
#pragma unroll
      for (int t = 0; t < PF; t += 2) {
        const int t1 = t + 1 < PF ? t + 1 : t;
        if constexpr (WIDE) {
          // The packed pair as loaded; slots past the batch count as (1, 1).
          const uint32_t lo = live[t] ? 0u : 0xffffu, hi = live[t1] ? 0u : 0xffff0000u;
          const uint32_t one2 = kOne | (kOne << 16);
          fast_quick_add<TT>(fq, (sv[t >> 1] & ~(lo | hi)) | (one2 & (lo | hi)),
                             (bv[t >> 1] & ~(lo | hi)) | (one2 & (lo | hi)));
        } else {
          const uint32_t sa = live[t] ? sv[t] : kOne, ba = live[t] ? bv[t] : kOne;
          const uint32_t sb = live[t1] ? sv[t1] : kOne, bb = live[t1] ? bv[t1] : kOne;
          fast_quick_add<TT>(fq, sa | (sb << 16), ba | (bb << 16));
        }
      }
      bool fast = ballot(!fast_quick_ok<TT>(fq)) == 0;
      if (!fast) {
        bool ok = true;
#pragma unroll
        for (int t = 0; t < PF; ++t) ok &= !live[t] || fast_ok_bits<TT>(sval(t) & 0xffffu, bval(t) & 0xffffu);
        fast = ballot(!ok) == 0;
      }
      // 2d. Multiply: A row m = lane & 15 (rows past the pass read row np-1:
      //     their outputs are never stored).
      const int m = min(r, np - 1);
      const unsigned char* xrowp = xw + m * RB;
#pragma unroll
      for (int t = 0; t < PF; ++t)
        if (t < nb) {
          acc = fast ? dec_step<TT, BITS, true>(wq[t], sval(t), bval(t), xrowp + t * 256, m, acc)
                     : dec_step<TT, BITS, false>(wq[t], sval(t), bval(t), xrowp + t * 256, m, acc);
        }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();  // the next batch restages this wave's region
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    for (int b0 = 0; b0 < nst; b0 += bmax) {
      const int nb = min(bmax, nst - b0);
      if (nb > 4) batch(b0, nb, std::integral_constant<int, 8>{});
      else if (nb > 2) batch(b0, nb, std::integral_constant<int, 4>{});
      else if (nb > 1) batch(b0, nb, std::integral_constant<int, 2>{});
      else batch(b0, nb, std::integral_constant<int, 1>{});
    }
    // 3. A column block's K parts in part order; element i of lane (r, g)
    //    is pass row 4g + i.
    if constexpr (KW > 1) {
      *reinterpret_cast<f32x4*>(red + (wave * 64 + lane) * 4) = acc;
      __syncthreads();
    }
    if (kw == 0 && n0 + r < n) {
      f32x4 v = acc;
#pragma unroll
      for (int i = 1; i < KW; ++i) v = v + *reinterpret_cast<const f32x4*>(red + ((wave + i) * 64 + lane) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mm = 4 * g + i;
        if (mm < np) {
          const int row = rlist[p0 + mm];
          y[(size_t)row * n + n0 + r] = ((lvmask >> row) & 1) ? TT::from_f32(v[i]) : (uint16_t)0;
        }
      }
    }
    if constexpr (KW > 1) __syncthreads();
  }
}

template <typename TT, int BITS, int KW, bool DENSE, bool WIDE>
hipError_t launch_dec(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                      const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                      unsigned int* status) {
  const int S = (k + 127) / 128;
  const int steps_w = (S + KW - 1) / KW;
  const int rows_max = DENSE ? std::min(kDensePass, n_rows) : std::min(kDecPass, n_rows);
  const int slots = DENSE ? (n_rows + rows_max - 1) / rows_max : n_rows;
  const size_t lds = gather_decode_lds(rows_max, k, KW);
  if (lds > 64 * 1024) {
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&gather_decode_kernel<TT, BITS, KW, DENSE, WIDE>);
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
  const int cols = 16 * (kDecWaves / KW);
  hipLaunchKernelGGL((gather_decode_kernel<TT, BITS, KW, DENSE, WIDE>),
                     dim3((unsigned)((n + cols - 1) / cols), (unsigned)slots), dim3(64 * kDecWaves), lds, s, q.w,
                     static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                     static_cast<const uint16_t*>(x), x_rows, lhs, rhs, n_rows, static_cast<uint16_t*>(y), n_experts,
                     n, k, gs_shift, (int)sorted, rows_max, steps_w, status);
  return hipGetLastError();
}

template <typename TT, int BITS, bool DENSE>
hipError_t launch_dec_w(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                        const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                        unsigned int* status, bool pad_exact) {
  const int slots = DENSE ? (n_rows + kDensePass - 1) / kDensePass : n_rows;
  int kw = gather_decode_kw(slots, n, k, DENSE);
  if (pad_exact && kw == 2) kw = 4;
  // Group size 64 with an even number of groups per row (every column's
  // row of scales starts on a 32-bit word): the form with wide (scale,
  // bias) loads.
  auto go = [&](auto widec) {
    constexpr bool W = decltype(widec)::value;
    if (kw == 4)
      return launch_dec<TT, BITS, 4, DENSE, W>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, status);
    if (kw == 2)
      return launch_dec<TT, BITS, 2, DENSE, W>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, status);
    return launch_dec<TT, BITS, 1, DENSE, W>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, status);
  };
  if (q.gs == 64 && ((k / 64) & 1) == 0) return go(std::true_type{});
  return go(std::false_type{});
}

template <bool DENSE>
hipError_t launch_dec_any(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                          const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                          unsigned int* status, bool pad_exact = false) {
  auto go = [&](auto tt, auto bits) {
    return launch_dec_w<decltype(tt), decltype(bits)::value, DENSE>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts,
                                                                    n, k, sorted, status, pad_exact);
  };
  if (q.dtype == CPQ_DTYPE_BF16) {
    if (q.bits == 4) return go(BF16{}, std::integral_constant<int, 4>{});
    if (q.bits == 8) return go(BF16{}, std::integral_constant<int, 8>{});
  }
  if (q.dtype == CPQ_DTYPE_F16) {
    if (q.bits == 4) return go(F16{}, std::integral_constant<int, 4>{});
    if (q.bits == 8) return go(F16{}, std::integral_constant<int, 8>{});
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Waves of a workgroup splitting K (the other factor of 4 splits columns),
// among the splits that keep the grid (column blocks x slots) within what
// the CUs hold at once, about 4 workgroups each, since every workgroup pays
// the same chain of dependent round trips (routing, weights and activations,
// sum).  The dense form takes the most such waves (its padded and unpadded
// K must choose alike); the routed form the split with the fewest steps per
// wave plus one per part (each part adds a share of the LDS sum and a wave
// that may be left short): config 5's down projection at one token (6
// steps) runs 5.47 us with 2 parts against 5.79 with 4.
int gather_decode_kw(int n_rows, int n, int k, bool dense) {
  const int forced = env_int("CPQ_DEC_KW", 0);  // tuning hook: 1, 2 or 4
  if (forced == 1 || forced == 2 || forced == 4) return forced;
  const long blocks = (n + 15) / 16;
  const int S = (k + 127) / 128;
  int best = 1, best_cost = S + 1;
  for (int kw = 4; kw > 1; kw /= 2) {
    const long wgs = (long)n_rows * ((blocks + (4 / kw) - 1) / (4 / kw));
    if (wgs > 1024) continue;
    if (dense) return kw;
    const int cost = (S + kw - 1) / kw + kw;
    if (cost < best_cost) {
      best_cost = cost;
      best = kw;
    }
  }
  return best;
}

size_t gather_decode_lds(int rows_max, int k, int kw) {
  const int S = (k + 127) / 128;
  const int steps_w = (S + kw - 1) / kw;
  return (size_t)kDecWaves * rows_max * std::min(steps_w, kDecPF) * 256 + (size_t)kDecWaves * 256 * sizeof(float) +
         kDecMaxRows * sizeof(int);
}

bool gather_decode_supported(const QuantArgs& q, int x_rows, int n_rows, int n, int k) {
  if (q.bits != 4 && q.bits != 8) return false;
  if (n_rows < 1 || n_rows > kDecMaxRows) return false;
  if (x_rows < 1 || (uint64_t)x_rows * (uint64_t)k * 2u >= (1ull << 31)) return false;  // x through one range
  if (q.gs != 32 && q.gs != 64 && q.gs != 128) return false;
  if (k % 128 != 0 || k < 128) return false;
  if ((uint64_t)n * (uint64_t)k * q.bits / 8 >= (1ull << 31) - (1ull << 20)) return false;
  if ((uint64_t)n * (uint64_t)(k / q.gs) * 2 >= (1ull << 31)) return false;
  return gather_decode_lds(std::min(kDecPass, n_rows), k, gather_decode_kw(n_rows, n, k, false)) <=
         (size_t)160 * 1024 - 1024;
}

hipError_t launch_gather_decode(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                                const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                                unsigned int* status) {
  return launch_dec_any<false>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, status);
}

bool dense_small_supported(const QuantArgs& q, int m, int n, int k) {
  if (q.bits != 4 && q.bits != 8) return false;
  if (q.dtype != CPQ_DTYPE_BF16 && q.dtype != CPQ_DTYPE_F16) return false;
  if (m < 1 || m > kDecMaxRows || (uint64_t)m * (uint64_t)k * 2u >= (1ull << 31)) return false;
  if (q.gs != 32 && q.gs != 64 && q.gs != 128) return false;
  if (k < q.gs || k % q.gs != 0) return false;  // whole groups; a partial last step is masked
  if ((uint64_t)n * (uint64_t)k * q.bits / 8 >= (1ull << 31) - (1ull << 20)) return false;
  if ((uint64_t)n * (uint64_t)(k / q.gs) * 2 >= (1ull << 31)) return false;
  const int slots = (m + kDensePass - 1) / kDensePass;
  return gather_decode_lds(std::min(kDensePass, m), k, gather_decode_kw(slots, n, k, true)) <= (size_t)160 * 1024 - 1024;
}

hipError_t launch_dense_small(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                              bool pad_exact) {
  return launch_dec_any<true>(s, q, x, m, nullptr, nullptr, m, y, 1, n, k, false, nullptr, pad_exact);
}

}  // namespace cpq
