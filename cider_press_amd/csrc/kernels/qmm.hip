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
#include <algorithm>

#include <cstdlib>

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

// ---------------------------------------------------------------------------
// Streaming prefill kernel (K % 128 == 0, 4/8-bit).
//
// Workgroup tile 128 (M) x 64 (N); its 4 waves are 2 N-halves x 2 K-halves,
// each wave owning a 128 x 32 tile (four 32x32 accumulators).  The matrix
// work per weight is then 128 MACs, enough to keep the VALU dequantization
// (one W column dequantized exactly once per workgroup, by the wave that
// owns it) below the MFMA time.  K advances in stages of 128: the K-half kh
// of a wave takes k in [128s + 64kh, 128s + 64kh + 64).
//   X: a ring of NSX LDS slots, each the 128 x 128 activation stage, filled by
//      global_load_lds_dwordx4 (no VGPRs), rows of 256 B with 16-B columns
//      XOR-swizzled by row (conflict-free ds_read_b128), NSX-1 stages ahead;
//   W: each lane streams the 32-element chunk of its column for its K-half
//      straight into registers, NSX-1 stages ahead, and dequantizes it into
//      the four MFMA B operands of the stage;
//   one s_barrier per stage; the two K-halves are summed through LDS at the
//      end.  Workgroups are ordered so the M-tiles sharing a W slab land on
//      the same XCD (same L2).
// MFMA 32x32x16 k mapping: step t, lane group h = lane/32, element j <->
// k = 128s + 64kh + 32h + 8t + j (the lane group's 32 k are one W chunk).
// ---------------------------------------------------------------------------

constexpr int SBM = 128, SBN = 64, SBK = 128;
constexpr int NSX = 4;                           // LDS ring slots
constexpr int SLOT_BYTES = SBM * SBK * 2;        // 32 KiB
constexpr int AHEAD = NSX - 1;                   // stages issued ahead

template <int BITS>
struct StreamCfg {
  static constexpr int WLOADS = BITS * 4 / 16;  // 16-B loads per chunk
  static constexpr int VM = 8 + WLOADS + 2;      // VMEM instructions issued per stage
};

struct StreamGeom {
  const uint32_t* wrow;
  const uint16_t* srow;
  const uint16_t* brow;
  const uint16_t* xsrc[8];
  int S, gs_shift, kh, hh, wave;
};

template <int BITS>
__device__ __forceinline__ void stream_issue(const StreamGeom& g, unsigned char* smem, int s,
                                             uint32_t* wdst, uint32_t& sb) {
  const int sc = min(s, g.S - 1);  // tail stages re-load the last stage (never consumed)
  unsigned char* slot = smem + (size_t)(s % NSX) * SLOT_BYTES;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    __builtin_amdgcn_global_load_lds(g.xsrc[j] + (size_t)sc * SBK, slot + (g.wave * 8 + j) * 1024, 16, 0, 0);
  const int c = 4 * sc + 2 * g.kh + g.hh;
  load_chunk<BITS>(g.wrow, (size_t)c, wdst);
  const int gi = (c << 5) >> g.gs_shift;
  sb = (uint32_t)g.srow[gi] | ((uint32_t)g.brow[gi] << 16);
}

template <typename TT, int BITS, bool FAST>
__device__ __forceinline__ void stream_loop(const StreamGeom& g, unsigned char* smem,
                                            uint32_t (&wbuf)[AHEAD][BITS], uint32_t (&sbuf)[AHEAD],
                                            f32x16 (&acc)[4], int lane) {
  const int l32 = lane & 31, csw = l32 & 15;
  for (int s0 = 0; s0 < g.S; s0 += AHEAD) {
#pragma unroll
    for (int p = 0; p < AHEAD; ++p) {
      const int s = s0 + p;
      if (s < g.S) {  // uniform
        // Stage s (X DMA, W chunk, scale/bias) is complete once only the
        // loads of the AHEAD-1 later stages can still be in flight.
        if constexpr (StreamCfg<BITS>::VM * (AHEAD - 1) == 22)
          asm volatile("s_waitcnt vmcnt(22)" ::: "memory");
        else
          asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        uint32_t cur[BITS];
#pragma unroll
        for (int i = 0; i < BITS; ++i) cur[i] = wbuf[p][i];
        const uint32_t sbv = sbuf[p];
        stream_issue<BITS>(g, smem, s + AHEAD, wbuf[p], sbuf[p]);

        const float sf = TT::to_f32((uint16_t)(sbv & 0xffffu));
        const float bf = TT::to_f32((uint16_t)(sbv >> 16));
        const float s16 = sf * 0.0625f;
        const float c0 = FAST ? fmaf(-1024.f, sf, bf) : 0.f;
        const float c1 = FAST ? fmaf(-64.f, sf, bf) : 0.f;
        const unsigned char* slot = smem + (size_t)(s % NSX) * SLOT_BYTES;
        u32x4 bop[4];
        bop[0] = dequant_slice_nat<TT, BITS, FAST, 0>(cur, sf, s16, bf, c0, c1);
        bop[1] = dequant_slice_nat<TT, BITS, FAST, 1>(cur, sf, s16, bf, c0, c1);
        bop[2] = dequant_slice_nat<TT, BITS, FAST, 2>(cur, sf, s16, bf, c0, c1);
        bop[3] = dequant_slice_nat<TT, BITS, FAST, 3>(cur, sf, s16, bf, c0, c1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int colx = (8 * g.kh + 4 * g.hh + t) ^ csw;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4 a = *reinterpret_cast<const u32x4*>(slot + (32 * i + l32) * 256 + colx * 16);
            acc[i] = Mfma32<TT>::run(a, bop[t], acc[i]);
          }
        }
      }
    }
  }
}

template <typename TT, int BITS>
__global__ __launch_bounds__(256) void qmm_stream_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int m, int n,
                                                         int k, int gs_shift, int tiles_m,
                                                         int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nh = wave & 1, kh = wave >> 1, hh = lane >> 5, l32 = lane & 31;

  // XCD-aware tile order: consecutive linear ids (same XCD) walk M first.
  const int nwg = tiles_m * tiles_n;
  int lin = blockIdx.x;
  if ((nwg & 7) == 0) lin = (lin & 7) * (nwg >> 3) + (lin >> 3);
  const int mt = lin % tiles_m, nt = lin / tiles_m;
  const int row0 = mt * SBM, col0 = nt * SBN;
  const int G = k >> gs_shift;

  // 1. Fast-path vote over the workgroup's 64 columns: loads first.
  constexpr int VOTE_SLOTS = 8;
  uint32_t vs[VOTE_SLOTS], vb[VOTE_SLOTS];
  const int vcount = SBN * G;
#pragma unroll
  for (int t = 0; t < VOTE_SLOTS; ++t) {
    const int i = tid + 256 * t;
    vs[t] = vb[t] = 0u;
    if (i < vcount) {
      const int cc = min(col0 + i / G, n - 1);
      const size_t off = (size_t)cc * G + (i % G);
      vs[t] = scales[off];
      vb[t] = biases[off];
    }
  }

  // 2. Stream prologue.
  StreamGeom g;
  const int col = min(col0 + 32 * nh + l32, n - 1);
  g.wrow = w + (size_t)col * ((size_t)k * BITS / 32);
  g.srow = scales + (size_t)col * G;
  g.brow = biases + (size_t)col * G;
  g.S = k / SBK;
  g.gs_shift = gs_shift;
  g.kh = kh;
  g.hh = hh;
  g.wave = wave;
  // X DMA: this wave fills blocks 8*wave .. 8*wave+7 (1 KiB = 4 rows each) of a
  // slot; lane i of block b lands at row 4b + i/16, physical 16-B column i%16,
  // which holds logical column (i%16) ^ (row%16).
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = (wave * 8 + j) * 4 + (lane >> 4);
    const int c = (lane & 15) ^ (rr & 15);
    const int grow = min(row0 + rr, m - 1);
    g.xsrc[j] = x + (size_t)grow * k + c * 8;
  }
  uint32_t wbuf[AHEAD][BITS];
  uint32_t sbuf[AHEAD];
#pragma unroll
  for (int p = 0; p < AHEAD; ++p) stream_issue<BITS>(g, smem, p, wbuf[p], sbuf[p]);

  // 3. Finish the vote (its loads are older than the stream's).
  bool ok = true;
#pragma unroll
  for (int t = 0; t < VOTE_SLOTS; ++t) ok &= fast_ok_bits<TT>(vs[t], vb[t]);
  for (int i = tid + 256 * VOTE_SLOTS; i < vcount; i += 256) {
    const int cc = min(col0 + i / G, n - 1);
    const size_t off = (size_t)cc * G + (i % G);
    ok &= fast_ok_bits<TT>(scales[off], biases[off]);
  }
  const bool fast = __syncthreads_and(ok);

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  if (fast)
    stream_loop<TT, BITS, true>(g, smem, wbuf, sbuf, acc, lane);
  else
    stream_loop<TT, BITS, false>(g, smem, wbuf, sbuf, acc, lane);

  // 4. Sum the two K-halves: kh = 1 waves park their tiles in LDS.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  float* park = reinterpret_cast<float*>(smem) + nh * (4 * 16 * 64);
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) park[(i * 16 + e) * 64 + lane] = acc[i][e];
  }
  __syncthreads();
  if (kh == 0) {
    const int gcol = col0 + 32 * nh + l32;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = acc[i][e] + park[(i * 16 + e) * 64 + lane];
        const int grow = row0 + 32 * i + 8 * (e >> 2) + 4 * hh + (e & 3);
        if (grow < m && gcol < n) y[(size_t)grow * n + gcol] = TT::from_f32(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Staged prefill kernel (4/8-bit, K % 1024 == 0).
//
// Workgroup tile 128 (M) x 64 (N), K in stages of 128.  The activation stage
// (128 rows x 128 k, 32 KiB) is copied into a ring of LDS slots with
// buffer_load_dwordx4 ... lds, 3 stages ahead.  Each copy instruction moves
// 4 rows x 256 contiguous bytes, so it needs 4 address translations; a
// row-per-lane load in MFMA layout would need 16, and the L1 TLB serialises
// translations (measured: it, not bandwidth, bounds such loads).  Rows keep
// their 16-byte chunks XOR-swizzled by row, so the MFMA-layout ds_read_b128
// is conflict-free.
// Wave w owns the whole 128 x 64 tile for the k-slice [32w, 32w+32) of every
// stage, so each staged activation byte is read from LDS exactly once and
// each weight is dequantized once per workgroup:
//   A: 8 x ds_read_b128 (row 16i + l%16, k 8(l/16)..+8 of the slice);
//   W: 4 x (BITS/4) words per lane loaded straight into registers 7 stages
//      ahead (lane l: word(s) l/16 of the slice's chunk of column 16j + l%16);
//   32 v_mfma_f32_16x16x32 per stage, column block by column block, each
//   block followed by the dequantization (natural k order) of that column's
//   B operand for the next stage, which overlaps the next block's MFMAs.
// One s_barrier per stage (the slot about to be refilled must have been read
// by every wave); the 4 K-partial tiles are summed through LDS at the end.
// MFMA 16x16x32 layout: A[m][k] lane m + 16(k/8), B[k][n] lane n + 16(k/8),
// element k%8; D[m][n] lane n + 16(m/4), element m%4.
// ---------------------------------------------------------------------------

constexpr int QBM = 128, QBN = 64, QBK = 128;
constexpr int QSLOT = QBM * QBK * 2;           // 32 KiB
constexpr int QRW = 8;                         // weight register ring
constexpr int QMAX_GROUPS = 256;               // groups per row the staged kernel accepts
constexpr int QEPI_MAX = 4 * 2 * 64 * (64 + 4) * 4;  // largest epilogue (MH = 2): 139264 B

struct StageGeom {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xoff[8];  // DMA source offset of this lane for its copy block j (stage 0)
  uint32_t woff[4];  // weight word offset (bytes) of column block j (stage 0)
  uint32_t a_off;    // byte offset of this lane's A fragment (i = 0) within a slot
  uint32_t c_off;    // byte offset of this lane's constants (group 0) in LDS
  unsigned char* smem;
  int wave, kw, gs_shift, S;
};

// Ring slot of stage s; s0 (the 8-stage block base) is a multiple of 8, so
// for NSX dividing 8 the slot is static.
template <int NSX, int P>
__device__ __forceinline__ int stage_slot(int s) {
  if constexpr (8 % NSX == 0) return P % NSX;
  return s % NSX;
}

template <int BITS, int NSX, int MH>
__device__ __forceinline__ void stage_dma(const StageGeom& g, int s, int slot_index) {
  unsigned char* slot = g.smem + (size_t)slot_index * QSLOT;
#pragma unroll
  for (int j = 0; j < 8 / MH; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        g.xr, (__attribute__((address_space(3))) void*)(slot + (g.wave * (8 / MH) + j) * 1024), 16,
        g.xoff[j], s * (QBK * 2), 0, 0);
}

template <int BITS>
__device__ __forceinline__ void stage_w(const StageGeom& g, int s, uint32_t (&wb)[4][BITS / 4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (BITS == 4) {
      wb[j][0] = __builtin_amdgcn_raw_buffer_load_b32(g.wr, g.woff[j], s * 16 * BITS, 0);
    } else {
      const u32x2 t =
          __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(g.wr, g.woff[j], s * 16 * BITS, 0));
      wb[j][0] = t.x;
      wb[j][1] = t.y;
    }
  }
}

// Raw constants of stage s: (s | b << 16) of the four column blocks.
__device__ __forceinline__ u32x4 stage_consts(const StageGeom& g, int s) {
  const int grp = (s * QBK + 32 * g.kw) >> g.gs_shift;
  return *reinterpret_cast<const u32x4*>(g.smem + g.c_off + (size_t)grp * 256);
}

template <typename TT, int BITS, bool FAST>
__device__ __forceinline__ u32x4 stage_dequant(const uint32_t (&wb)[BITS / 4], uint32_t sbv) {
  const float sf = TT::to_f32((uint16_t)(sbv & 0xffffu)), bf = TT::to_f32((uint16_t)(sbv >> 16));
  const float c0 = FAST ? fmaf(-1024.f, sf, bf) : 0.f;
  const float c1 = FAST ? fmaf(-64.f, sf, bf) : 0.f;
  return dequant_slice_nat<TT, BITS, FAST, 0>(wb, sf, sf * 0.0625f, bf, c0, c1);
}

// VMEM instructions issued after stage s+1's copies up to the start of stage
// s -- the vmcnt that proves those copies complete.  Stage t issues 8 copies
// (for t+3) when t+3 < S, then 4 weight loads (for t+7) when t+7 < S; the
// prologue issues in the same pattern.  Only the last 8 stages (TAIL,
// P = s - (S-8)) differ from the steady 4 + 12.
template <int MH, bool TAIL, int P>
constexpr int stage_vmcnt() {
  if constexpr (!TAIL) {
    return 8 + 8 / MH;
  } else {
    return 4 * (P <= 2) + (8 / MH) * (P <= 5) + 4 * (P <= 1);
  }
}

// Stage s = s0 + P.  On entry a[P & 1] holds stage s's A fragments and bop
// its B operands.  The stage proves stage s+1's copies complete (own vmcnt,
// then the barrier for the other waves'), refills the slot of stage s-1
// (copies for s+3) and the weight ring (s+7), reads stage s+1's fragments
// into a[(P + 1) & 1], and runs its MFMAs with the next stage's
// dequantization between the column blocks.
template <typename TT, int BITS, int NSX, int MH, bool FAST, bool TAIL, int P>
__device__ __forceinline__ void stage_step(const StageGeom& g, int s, uint32_t (&wv)[QRW][4][BITS / 4],
                                           u32x4 (&a)[2][8 / MH], u32x4 (&bop)[4],
                                           f32x4 (&acc)[8 / MH][4]) {
  constexpr int NI = 8 / MH;
  constexpr bool DMA = !TAIL || P + 3 < 8;
  constexpr bool WLD = !TAIL || P + 7 < 8;
  constexpr bool NEXT = !TAIL || P + 1 < 8;
  if constexpr (NEXT) {
    wait_vmcnt<stage_vmcnt<MH, TAIL, P>()>();
    __builtin_amdgcn_s_barrier();
  }
  if constexpr (DMA) stage_dma<BITS, NSX, MH>(g, s + 3, stage_slot<NSX, (P + 3) % 8>(s + 3));
  if constexpr (WLD) stage_w<BITS>(g, s + 7, wv[(P + 7) % QRW]);
  u32x4 cn = {0u, 0u, 0u, 0u};
  if constexpr (NEXT) {
    const unsigned char* slot = g.smem + (size_t)stage_slot<NSX, (P + 1) % 8>(s + 1) * QSLOT + g.a_off;
#pragma unroll
    for (int i = 0; i < NI; ++i) a[(P + 1) & 1][i] = *reinterpret_cast<const u32x4*>(slot + i * 4096);
    cn = stage_consts(g, s + 1);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < NI; ++i) acc[i][j] = Mfma16<TT>::run(a[P & 1][i], bop[j], acc[i][j]);
    if constexpr (NEXT) bop[j] = stage_dequant<TT, BITS, FAST>(wv[(P + 1) % QRW][j], cn[j]);
  }
}

template <typename TT, int BITS, int NSX, int MH, bool FAST, bool TAIL, int P = 0>
__device__ __forceinline__ void stage_eight(const StageGeom& g, int s0, uint32_t (&wv)[QRW][4][BITS / 4],
                                            u32x4 (&a)[2][8 / MH], u32x4 (&bop)[4],
                                            f32x4 (&acc)[8 / MH][4]) {
  if constexpr (P < 8) {
    stage_step<TT, BITS, NSX, MH, FAST, TAIL, P>(g, s0 + P, wv, a, bop, acc);
    stage_eight<TT, BITS, NSX, MH, FAST, TAIL, P + 1>(g, s0, wv, a, bop, acc);
  }
}

template <typename TT, int BITS, int NSX, int MH, bool FAST>
__device__ __forceinline__ void stage_loop(const StageGeom& g, uint32_t (&wv)[QRW][4][BITS / 4],
                                           f32x4 (&acc)[8 / MH][4]) {
  // Stage 0's copies are complete: the constant staging waited for every
  // earlier load and the vote ended in a barrier.
  u32x4 a[2][8 / MH], bop[4];
  const unsigned char* slot = g.smem + g.a_off;
#pragma unroll
  for (int i = 0; i < 8 / MH; ++i) a[0][i] = *reinterpret_cast<const u32x4*>(slot + i * 4096);
  const u32x4 c0 = stage_consts(g, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) bop[j] = stage_dequant<TT, BITS, FAST>(wv[0][j], c0[j]);
  int s0 = 0;
  for (; s0 < g.S - 8; s0 += 8) stage_eight<TT, BITS, NSX, MH, FAST, false>(g, s0, wv, a, bop, acc);
  stage_eight<TT, BITS, NSX, MH, FAST, true>(g, s0, wv, a, bop, acc);
}

template <typename TT, int BITS, int NSX, int MH>
__global__ __launch_bounds__(256 * MH) __attribute__((amdgpu_waves_per_eu(MH, MH))) void qmm_staged_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
    int m, int n, int k, int gs_shift, int tiles_m, int tiles_n, int sb_vec) {
  constexpr int NT = 256 * MH;   // threads
  constexpr int NI = 8 / MH;     // 16-row blocks per wave
  constexpr int RW = 128 / MH;   // rows per wave
  constexpr int EPI = RW + 4;    // epilogue floats per lane (padded)
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave & 3, mh = wave >> 2;
  const int l16 = lane & 15, lg = lane >> 4;

  // Tile order: each XCD (linear ids congruent mod 8) gets a contiguous run
  // of tiles, N fastest, so its workgroups share one activation panel in L2.
  const int nwg = tiles_m * tiles_n;
  int v = blockIdx.x;
  if ((nwg & 7) == 0) v = (v & 7) * (nwg >> 3) + (v >> 3);
  const int mt = v / tiles_n, nt = v % tiles_n;
  const int row0 = mt * QBM, col0 = nt * QBN;
  const int G = k >> gs_shift;

  StageGeom g;
  g.smem = smem;
  g.wave = wave;
  g.kw = kw;
  g.gs_shift = gs_shift;
  g.S = k / QBK;
  g.xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);
  g.wr = __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * (uint32_t)k / 8u * (uint32_t)BITS),
                                           0x00020000);
  // Copy block b = NI*wave + j holds rows 4b .. 4b+3; lane i lands at row
  // 4b + i/16, physical chunk i%16, which holds logical chunk (i%16)^(row%16).
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int rr = (wave * NI + j) * 4 + (lane >> 4);
    const int c = (lane & 15) ^ (rr & 15);
    const int grow = min(row0 + rr, m - 1);
    g.xoff[j] = ((uint32_t)grow * (uint32_t)k + (uint32_t)(c * 8)) * 2u;
  }
  // A fragment of lane (m = l16, lg): row RW*mh + 16i + m, logical chunk 4*kw + lg.
  g.a_off = (uint32_t)((RW * mh + l16) * 256 + (((4 * kw + lg) ^ l16) * 16));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = min(col0 + 16 * j + l16, n - 1);
    g.woff[j] = (uint32_t)col * ((uint32_t)k / 8u * BITS) + (uint32_t)(kw * 4 * BITS) + (uint32_t)(lg * BITS);
  }
  const uint32_t cst_base = (uint32_t)NSX * QSLOT;
  g.c_off = cst_base + (uint32_t)l16 * 16;

  // 1. Prologue loads in the steady-state issue pattern: W for stages 0..3,
  //    then (copies of stage t, W of stage t+4) for t = 0..2.
  uint32_t wv[QRW][4][BITS / 4];
#pragma unroll
  for (int t = 0; t < 4; ++t) stage_w<BITS>(g, t, wv[t]);
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    stage_dma<BITS, NSX, MH>(g, t, t);
    stage_w<BITS>(g, t + 4, wv[t + 4]);
  }

  // 2. Raw per-(column, group) constants into LDS, [(g*16 + n)*4 + j] for
  //    column col0 + 16j + n; the workgroup votes on the fast dequantization.
  //    Vector path: thread (block u, column c = tid % 64) loads 8 groups of
  //    its column per block, all blocks' loads in flight together.
  uint32_t* cst = reinterpret_cast<uint32_t*>(smem + cst_base);
  bool ok = true;
  auto put = [&](int c, int gi, uint32_t sv, uint32_t bv) { cst[(gi * 16 + (c & 15)) * 4 + (c >> 4)] = sv | (bv << 16); };
  if (sb_vec) {
    constexpr int MAXB = QMAX_GROUPS / 8 / (NT / 64);  // 8-group blocks per thread
    const int c = tid & 63, col = min(col0 + c, n - 1);
    const int nblk = G >> 3;
    u32x4 sv[MAXB], bv[MAXB];
#pragma unroll
    for (int u = 0; u < MAXB; ++u) {
      const int gb = (tid >> 6) + (NT / 64) * u;
      if (gb < nblk) {
        sv[u] = *reinterpret_cast<const u32x4*>(scales + (size_t)col * G + gb * 8);
        bv[u] = *reinterpret_cast<const u32x4*>(biases + (size_t)col * G + gb * 8);
      }
    }
    // Packed exponent check over the thread's blocks; the exact predicate
    // per group only when that one does not clear them.
    FastQuick fq;
    fast_quick_init(fq);
#pragma unroll
    for (int u = 0; u < MAXB; ++u) {
      const int gb = (tid >> 6) + (NT / 64) * u;
      if (gb < nblk) {
#pragma unroll
        for (int q = 0; q < 4; ++q) fast_quick_add<TT>(fq, sv[u][q], bv[u][q]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          put(c, gb * 8 + e, (e & 1) ? sv[u][e >> 1] >> 16 : sv[u][e >> 1] & 0xffffu,
              (e & 1) ? bv[u][e >> 1] >> 16 : bv[u][e >> 1] & 0xffffu);
      }
    }
    if (!fast_quick_ok<TT>(fq)) {
#pragma unroll
      for (int u = 0; u < MAXB; ++u) {
        const int gb = (tid >> 6) + (NT / 64) * u;
        if (gb < nblk) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            ok &= fast_ok_bits<TT>(sv[u][q] & 0xffffu, bv[u][q] & 0xffffu) &
                  fast_ok_bits<TT>(sv[u][q] >> 16, bv[u][q] >> 16);
        }
      }
    }
  } else {
    for (int it = tid; it < 64 * G; it += NT) {
      const int c = it & 63, gi = it >> 6;
      const size_t off = (size_t)min(col0 + c, n - 1) * G + gi;
      ok &= fast_ok_bits<TT>(scales[off], biases[off]);
      put(c, gi, scales[off], biases[off]);
    }
  }
  const bool fast = __syncthreads_and(ok);

  // 3. Stream K.
  f32x4 acc[NI][4];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (fast)
    stage_loop<TT, BITS, NSX, MH, true>(g, wv, acc);
  else
    stage_loop<TT, BITS, NSX, MH, false>(g, wv, acc);

  // 4. Sum the four K-partial tiles of each row half: every wave parks its
  //    tile, then thread (kw, mh, lane) adds up accumulator tiles
  //    NI*kw .. NI*kw+NI-1 of its lane over the four waves of its row half.
  __syncthreads();
  float* ep = reinterpret_cast<float*>(smem);
  {
    float* mine = ep + (wave * 64 + lane) * EPI;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<f32x4*>(mine + 4 * (i * 4 + j)) = acc[i][j];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NI; ++q) {
    const int t = NI * kw + q, i = t >> 2, j = t & 3;
    f32x4 sum = *reinterpret_cast<const f32x4*>(ep + ((4 * mh) * 64 + lane) * EPI + 4 * t);
#pragma unroll
    for (int w2 = 1; w2 < 4; ++w2)
      sum += *reinterpret_cast<const f32x4*>(ep + ((4 * mh + w2) * 64 + lane) * EPI + 4 * t);
    const int gcol = col0 + 16 * j + l16;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int grow = row0 + RW * mh + 16 * i + 4 * lg + e;
      if (grow < m && gcol < n) y[(size_t)grow * n + gcol] = TT::from_f32(sum[e]);
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
hipError_t launch_stream(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                         int k) {
  const size_t lds = (size_t)NSX * SLOT_BYTES;
  static const hipError_t attr = [] {
    const void* fn = reinterpret_cast<const void*>(&qmm_stream_kernel<TT, BITS>);
    hipFuncAttributes fa;
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(160 * 1024 - fa.sharedSizeBytes));
  }();
  if (attr != hipSuccess) return attr;
  const int tiles_m = (m + SBM - 1) / SBM, tiles_n = (n + SBN - 1) / SBN;
  hipLaunchKernelGGL((qmm_stream_kernel<TT, BITS>), dim3((unsigned)(tiles_m * tiles_n)), dim3(256), lds,
                     s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), m, n, k, shift_of(q.gs), tiles_m, tiles_n);
  return hipGetLastError();
}

// LDS ring depth of the staged kernel: 4 slots when the constants fit
// beside them in 160 KiB, else 3; 0 if not even that fits.
int staged_slots(int k, int gs) {
  const int G = k / gs;
  const int budget = 160 * 1024 - 256;  // minus __syncthreads_and's static LDS
  if (4 * QSLOT + G * 256 <= budget) return 4;
  if (3 * QSLOT + G * 256 <= budget) return 3;
  return 0;
}

// The staged kernel addresses X and W with 32-bit byte offsets.
bool staged_fits(int m, int n, int k, int gs, int bits) {
  const uint64_t xb = (uint64_t)m * k * 2, wb = (uint64_t)n * k * bits / 8;
  return k % 1024 == 0 && k / gs <= QMAX_GROUPS && staged_slots(k, gs) > 0 && xb < (1ull << 31) &&
         wb < (1ull << 31);
}

template <typename TT, int BITS, int NSX, int MH>
hipError_t launch_staged_n(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                           int k) {
  static const hipError_t attr = [] {
    const void* fn = reinterpret_cast<const void*>(&qmm_staged_kernel<TT, BITS, NSX, MH>);
    hipFuncAttributes fa;
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(160 * 1024 - fa.sharedSizeBytes));
  }();
  if (attr != hipSuccess) return attr;
  const int G = k / q.gs;
  const size_t epi = (size_t)4 * MH * 64 * (128 / MH + 4) * 4;
  const size_t lds = std::max((size_t)NSX * QSLOT + (size_t)G * 256, epi);
  const int sb_vec = (G % 8 == 0) && (reinterpret_cast<uintptr_t>(q.scales) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(q.biases) % 16 == 0);
  const int tiles_m = (m + QBM - 1) / QBM, tiles_n = (n + QBN - 1) / QBN;
  hipLaunchKernelGGL((qmm_staged_kernel<TT, BITS, NSX, MH>), dim3((unsigned)(tiles_m * tiles_n)),
                     dim3(256 * MH), lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), m, n, k, shift_of(q.gs), tiles_m, tiles_n, sb_vec);
  return hipGetLastError();
}

#ifndef CPQ_STAGED_MH
#define CPQ_STAGED_MH 1
#endif

template <typename TT, int BITS>
hipError_t launch_staged(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                         int k) {
  if (staged_slots(k, q.gs) == 4) return launch_staged_n<TT, BITS, 4, CPQ_STAGED_MH>(s, q, x, y, m, n, k);
  return launch_staged_n<TT, BITS, 3, CPQ_STAGED_MH>(s, q, x, y, m, n, k);
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  if constexpr (BITS == 4 || BITS == 8) {
    if (staged_fits(m, n, k, q.gs, BITS)) return launch_staged<TT, BITS>(s, q, x, y, m, n, k);
    if (k % SBK == 0) return launch_stream<TT, BITS>(s, q, x, y, m, n, k);
  }
  // Fill the chip: 128x128 tiles when they give at least ~2 workgroups per
  // CU, else 64-row tiles.
  const long tiles128 = (long)((m + 127) / 128) * ((n + 127) / 128);
  if (tiles128 >= 512) return launch_cfg<TT, BITS, 128, 128, 2, 2>(s, q, x, y, m, n, k);
  return launch_cfg<TT, BITS, 64, 128, 2, 2>(s, q, x, y, m, n, k);
}

}  // namespace

hipError_t launch_qmm_unsplit(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
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

// CPQ_QMM_WIDE=0 turns the wide-tile kernel off; CPQ_QMM_SPLIT=1|2|4 forces
// its K split.  Both are read per call (test and tuning hooks).
QmmPlan qmm_plan(const QuantArgs& q, int m, int n, int k, int cu_count, size_t scratch_cap) {
  const bool sb16 = ((reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases)) & 15u) == 0;
  // CPQ_QMM_DMA=0 turns the two-waves-per-SIMD kernel off (tuning hook).
  if (q.bits == 4 && sb16 && env_int("CPQ_QMM_DMA", 1) != 0) {
    const int forced = env_int("CPQ_QMM_SPLIT", 0);
    int split = forced > 0 ? (qmm_dma_fits(m, n, k, q.gs, q.bits, forced) ? forced : 0)
                           : qmm_dma_split(m, n, k, q.gs, q.bits, cu_count);
    for (; split > 1; split /= 2) {
      if (!qmm_dma_fits(m, n, k, q.gs, q.bits, split)) continue;
      const size_t need = qmm_dma_scratch_bytes(m, n, split);
      if (need <= scratch_cap) return QmmPlan{QmmKernel::Dma, split, need};
    }
    if (split == 1 && qmm_dma_fits(m, n, k, q.gs, q.bits, 1)) return QmmPlan{QmmKernel::Dma, 1, 0};
  }
  if (q.bits == 4 && sb16 && env_int("CPQ_QMM_WIDE", 1) != 0) {
    const int forced = env_int("CPQ_QMM_SPLIT", 0);
    int split = forced > 0 ? (qmm_wide_fits(m, n, k, q.gs, q.bits, forced) ? forced : 0)
                           : qmm_wide_split(m, n, k, q.gs, q.bits, cu_count);
    // A split needs its partial tiles in scratch; when they do not fit the
    // capacity, try smaller splits (a decision made from the shape and the
    // capacity only, the same eagerly and under graph capture).
    for (; split > 1; split /= 2) {
      if (!qmm_wide_fits(m, n, k, q.gs, q.bits, split)) continue;
      const size_t need = qmm_wide_scratch_bytes(m, n, split);
      if (need <= scratch_cap) return QmmPlan{QmmKernel::Wide, split, need};
    }
    if (split == 1 && qmm_wide_fits(m, n, k, q.gs, q.bits, 1)) return QmmPlan{QmmKernel::Wide, 1, 0};
  }
  return QmmPlan{QmmKernel::Unsplit, 1, 0};
}

hipError_t launch_qmm(hipStream_t s, const QmmPlan& plan, void* scratch, const QuantArgs& q, const void* x,
                      void* y, int m, int n, int k) {
  void* sp = plan.scratch_bytes ? scratch : nullptr;
  if (plan.kernel == QmmKernel::Dma) return launch_qmm_dma(s, q, x, y, m, n, k, plan.split, sp);
  if (plan.kernel == QmmKernel::Wide) return launch_qmm_wide(s, q, x, y, m, n, k, plan.split, sp);
  return launch_qmm_unsplit(s, q, x, y, m, n, k);
}

}  // namespace cpq
