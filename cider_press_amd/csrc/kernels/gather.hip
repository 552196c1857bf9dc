// Routed-expert quantized matmul, expert-major, for gfx950:
//   Y[r, :] = X[lhs[r], :] . dequant(W[rhs[r]])^T      (r < n_rows)
//
// Reference semantics: affine_gather_qmm_rhs / affine_gather_qmm_t
// (kernels-mlx/.../quantized.h:2092-2172, 2242-2436): each routed row is
// multiplied by its expert's weight, dequantized to T, fp32 accumulation.
//
// A workgroup (8 waves) owns one expert and one chunk of NC output columns.
// Per pass it gathers up to R = 16*MB of the rows routed to its expert (in row
// order: sorted routing by counting the rows below / at the expert in one
// pass, unsorted by per-64-row-block match counts, their prefix, and a ballot
// placement), stages those rows' activations in LDS once, and then streams
// the chunk's weights:
//   - wave w owns the 16-column slabs w, w+8, ... of the chunk; for each slab
//     it walks K in units of 4 chunks (lane l: column l%16, chunk 4u + l/16);
//     the unit's weights, (scale, bias) words and LDS offsets move by
//     wave-uniform amounts, so the loads take them in the scalar offset and
//     the step costs no address arithmetic beyond one add per LDS read;
//   - weights run 4 steps ahead of use and (scale, bias) words 4 to 8 steps
//     ahead, in register rings indexed by the unrolled step (no copies);
//   - each step is dequantized in registers (the exact single-FMA form when
//     the packed exponent check clears the wave's (scale, bias) words of the
//     load, else fmaf; the same bits either way) into four
//     v_mfma_f32_16x16x32 B operands and multiplied against the pass's
//     16-row activation blocks read from LDS;
//   - at a slab's last step its 16 x R tile is stored.
// The routing, the pass's activation rows and their loads go first (three
// dependent round trips on a memory system not yet loaded by the stream);
// the first weight steps are requested right after the activation loads.
// Activation layout in LDS: [unit][16-row block][row][16 slots of 16 bytes],
// slot s of row i stored at slot s ^ key(i % 16), key(r) = r with its 2-bit
// halves swapped, so that both lanes 16p .. 16p+15 and lanes p, p+4, ...,
// p+60 of an MFMA operand read touch 16 distinct slots (no bank conflicts).  Weights stream from HBM exactly once per pass and
// activations are read from L2 once per workgroup, so the kernel runs at the
// weight stream's rate for routings with up to R rows per expert (more rows:
// more passes).
#include <algorithm>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int GX_WAVES = 8;
constexpr int GX_THREADS = 64 * GX_WAVES;
constexpr int GX_PF = 4;                   // weight steps in flight per wave
constexpr int GX_UNROLL = 8;               // steps per loop iteration: two turns of the weight ring
constexpr int GX_XBYTES = 128 * 1024;      // LDS for the staged activation rows
constexpr int GX_MAXBLK = 1024;            // 64-row routing blocks (n_rows <= 65536)
constexpr int GX_COUNT_ROWS = 16 * GX_THREADS;  // sorted routing: counted in one pass up to this many rows
constexpr int GX_KEEP = 4;  // unsorted routing: 64-row blocks per wave counted in one round (2048 rows)
constexpr int GX_XITEMS = GX_XBYTES / 16 / GX_THREADS;  // staged 16-byte items per thread: all of a pass

struct GxShared {
  int cnt[GX_MAXBLK];  // unsorted routing: matches of this expert per 64-row block, then prefix
  unsigned long long keep[GX_WAVES][GX_KEEP];  // unsorted routing: match masks of each wave's first blocks
  int rows[64];        // routed rows of the pass (-1: none)
  int xrow[64];        // their activation rows (-1: none / invalid)
  uint32_t orow[64];   // byte offset of each pass row's output row in Y (past Y: not stored)
  int total, lo;
};

// A wave's position in its (slab, unit) steps; wave-uniform.
struct GxPos {
  int u, j;
  __device__ __forceinline__ void step(int units) {
    if (++u == units) {
      u = 0;
      ++j;
    }
  }
  __device__ __forceinline__ void skip(int n, int units) {  // n divides units
    u += n;
    if (u == units) {
      u = 0;
      ++j;
    }
  }
};

// (scale, bias) words per load: QS steps' groups of a lane's column (QS > 1:
// 16 or 8 bytes, the same for every lane of a column), or one 16-bit group
// per step (QS = 1).
template <int QS, int GSQ>
struct GxSbw {
  static constexpr int kWords = QS == 1 ? 1 : QS * 64 / GSQ;
  static_assert(QS == 1 || kWords == 2 || kWords == 4, "8- or 16-byte (scale, bias) loads");
};

// Register rings of one wave's stream: weights of GX_PF steps, (scale,
// bias) words of GX_UNROLL steps.
template <int BITS, int QS, int GSQ>
struct GxRing {
  static constexpr int kSb = GX_UNROLL / QS;
  static constexpr int kW = GxSbw<QS, GSQ>::kWords;
  uint32_t w[GX_PF][BITS];
  uint32_t s[kSb][kW], b[kSb][kW];
};

template <int BITS>
__device__ __forceinline__ void gx_wload(__amdgpu_buffer_rsrc_t wr, uint32_t voff, uint32_t soff,
                                         uint32_t (&dst)[BITS]) {
  static_assert(BITS == 4 || BITS == 8, "4- and 8-bit");
#pragma unroll
  for (int q = 0; q < BITS / 4; ++q) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff + 16u * q, soff, 0));
    dst[4 * q] = v.x;
    dst[4 * q + 1] = v.y;
    dst[4 * q + 2] = v.z;
    dst[4 * q + 3] = v.w;
  }
}

template <int QS, int GSQ, int W>
__device__ __forceinline__ void gx_sbload(__amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t br, uint32_t voff,
                                          uint32_t soff, uint32_t (&s)[W], uint32_t (&b)[W]) {
  if constexpr (W == 4) {
    const u32x4 sv = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, voff, soff, 0));
    const u32x4 bv = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(br, voff, soff, 0));
    s[0] = sv.x; s[1] = sv.y; s[2] = sv.z; s[3] = sv.w;
    b[0] = bv.x; b[1] = bv.y; b[2] = bv.z; b[3] = bv.w;
  } else if constexpr (W == 2) {
    const u32x2 sv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sr, voff, soff, 0));
    const u32x2 bv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(br, voff, soff, 0));
    s[0] = sv[0]; s[1] = sv[1];
    b[0] = bv[0]; b[1] = bv[1];
  } else {
    s[0] = __builtin_amdgcn_raw_buffer_load_b16(sr, voff, soff, 0);
    b[0] = __builtin_amdgcn_raw_buffer_load_b16(br, voff, soff, 0);
  }
}

// The 16-bit scale or bias of step I of a load for this lane (lane group g)
// as f32.  QS = 1: the loaded group.  GSQ = 64: groups 2(u+I) .. +1 of the
// load's first unit u are word I; this lane's is half g / 2 (`sel`).
// GSQ = 128: group u + I is word I / 2, half I % 2.
template <typename TT, int QS, int GSQ, int W>
__device__ __forceinline__ float gx_sbv(const uint32_t (&v)[W], int I, uint32_t sel) {
  if constexpr (QS == 1) {
    return TT::to_f32((uint16_t)v[0]);
  } else if constexpr (GSQ == 64) {
    const uint32_t word = v[I];
    if constexpr (Sig16<TT>::bf16)
      return __uint_as_float(__builtin_amdgcn_perm(word, word, sel));
    else
      return TT::to_f32((uint16_t)__builtin_amdgcn_perm(word, word, sel));
  } else {
    const uint32_t word = v[I >> 1];
    return TT::to_f32((uint16_t)((I & 1) ? word >> 16 : word & 0xffffu));
  }
}

// Byte selector of gx_sbv for lane group g (GSQ = 64): the 16-bit half
// g / 2 into the high half (bf16: the f32 bits) or the low half (f16).
template <typename TT>
__device__ __forceinline__ uint32_t gx_sb_sel(int g) {
  if constexpr (Sig16<TT>::bf16)
    return (g >> 1) ? 0x03020c0cu : 0x01000c0cu;
  else
    return (g >> 1) ? 0x0c0c0302u : 0x0c0c0100u;
}

// Where a wave's stream reads: the expert's weight and (scale, bias) tables
// as buffers, the lane's byte offsets at step 0 (its column's row; plus its
// chunk g for weights, and its group for QS = 1), the bytes between the
// wave's consecutive slabs and per unit.
struct GxSrc {
  __amdgpu_buffer_rsrc_t wr, sr, br;
  uint32_t wl, sl;
  uint32_t wslab, sslab;
  uint32_t wunit, sunit;
  uint32_t wlast, slast;  // uniform offsets of the last step's weights and (scale, bias) load
  __device__ __forceinline__ uint32_t woff(const GxPos& p) const { return p.j * wslab + p.u * wunit; }
  __device__ __forceinline__ uint32_t soff(const GxPos& p) const { return p.j * sslab + p.u * sunit; }
};

// The ring's first steps: weights of steps 0 .. GX_PF-1, (scale, bias) words
// of steps 0 .. GX_UNROLL-1.  On return `wpos` / `spos` are the positions of
// the next steps to load.  Every ring load is issued unconditionally (a step
// past the wave's last re-reads the last one), so the compiler counts the
// loads in flight exactly and never waits for more of them than it needs.
template <int BITS, int QS, int GSQ>
__device__ __forceinline__ void gx_fill(const GxSrc& src, GxRing<BITS, QS, GSQ>& ring, int T, int units,
                                        GxPos& wpos, GxPos& spos) {
  wpos = GxPos{0, 0};
  spos = GxPos{0, 0};
#pragma unroll
  for (int p = 0; p < GX_PF; ++p) {
    gx_wload<BITS>(src.wr, src.wl, p < T ? src.woff(wpos) : src.wlast, ring.w[p]);
    wpos.step(units);
  }
#pragma unroll
  for (int q = 0; q < GxRing<BITS, QS, GSQ>::kSb; ++q) {
    gx_sbload<QS, GSQ>(src.sr, src.br, src.sl, q * QS < T ? src.soff(spos) : src.slast, ring.s[q], ring.b[q]);
    spos.skip(QS, units);
  }
}

// Whether the single-FMA dequantization is exact for the (scale, bias)
// words of one load, per lane: lane group g checks word g % W of its
// column's words with the packed check (the lane groups of a column hold the
// same words); QS = 1: each lane its own group.  Sufficient, not necessary:
// steps it does not clear are dequantized with fmaf, the same bits.
template <typename TT, int QS, int W>
__device__ __forceinline__ void gx_fast_add(FastQuick& fq, const uint32_t (&s)[W], const uint32_t (&b)[W], int g) {
  // Words picked by masks, not by index: an array indexed by a lane value
  // would be kept in scratch memory.
  uint32_t sw, bw;
  if constexpr (QS == 1) {
    sw = s[0] | (s[0] << 16);
    bw = b[0] | (b[0] << 16);
  } else {
    const uint32_t m1 = 0u - (uint32_t)(g & 1);
    sw = s[0] ^ ((s[0] ^ s[1]) & m1);
    bw = b[0] ^ ((b[0] ^ b[1]) & m1);
    if constexpr (W == 4) {
      const uint32_t m2 = 0u - (uint32_t)((g >> 1) & 1);
      const uint32_t s23 = s[2] ^ ((s[2] ^ s[3]) & m1), b23 = b[2] ^ ((b[2] ^ b[3]) & m1);
      sw = sw ^ ((sw ^ s23) & m2);
      bw = bw ^ ((bw ^ b23) & m2);
    }
  }
  fast_quick_add<TT>(fq, sw, bw);
}

// What one step of a wave's stream needs besides the ring.
struct GxCtx {
  int T, units, my_slabs, g, mbl;
  uint32_t sel;
  uint32_t aoff[4];
  const unsigned char* xs;
  const uint32_t* orow;  // LDS: byte offsets of the pass's output rows
  int col0, n;
  __amdgpu_buffer_rsrc_t yr;
};

// GX_UNROLL steps t0 .. t0+GX_UNROLL-1 of the stream, straight-line code:
// no branch but the uniform one around a slab's stores, so the compiler's
// count of loads in flight stays exact.  Steps past the wave's last (the
// rounding of T up to a whole group) re-read the last step's words, compute
// on them and store nothing.  MBL of the MB 16-row blocks are multiplied:
// the ones that hold rows of the pass (each block read costs LDS bandwidth).
template <typename TT, int BITS, int MB, int MBL, bool FAST, int QS, int GSQ>
__device__ __forceinline__ void gx_group(const GxSrc& src, GxRing<BITS, QS, GSQ>& ring, GxPos& wpos, GxPos& spos,
                                         GxPos& cur, int t0, f32x4 (&acc)[MB], const GxCtx& cx) {
#pragma unroll
  for (int p = 0; p < GX_UNROLL; ++p) {
    const int t = t0 + p;
    constexpr int kSbSlots = GxRing<BITS, QS, GSQ>::kSb;
    const int q = (p / QS) % kSbSlots, I = p % QS;
    // This step's activation operands first: their LDS latency runs under
    // the dequantization instead of between the MFMAs.
    // (Up to two blocks: more would hold too many registers across the
    // dequantization.)
    constexpr bool kEarly = MBL <= 2;
    const uint32_t ub = (uint32_t)cur.u * (MB * 4096u);
    u32x4 a[4][MBL];
    if constexpr (kEarly) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int mb = 0; mb < MBL; ++mb)
          a[i][mb] = *reinterpret_cast<const u32x4*>(cx.xs + cx.aoff[i] + ub + mb * 4096);
    }
    const float sf = gx_sbv<TT, QS, GSQ>(ring.s[q], I, cx.sel);
    const float bf = gx_sbv<TT, QS, GSQ>(ring.b[q], I, cx.sel);
    const float s16 = sf * 0.0625f;
    const float c0 = FAST ? fmaf(-1024.f, sf, bf) : 0.f, c1 = FAST ? fmaf(-64.f, sf, bf) : 0.f;
    uint32_t(&wcur)[BITS] = ring.w[p % GX_PF];
    u32x4 bop[4];
    bop[0] = dequant_slice<TT, BITS, FAST, 0>(wcur, sf, s16, bf, c0, c1);
    bop[1] = dequant_slice<TT, BITS, FAST, 1>(wcur, sf, s16, bf, c0, c1);
    bop[2] = dequant_slice<TT, BITS, FAST, 2>(wcur, sf, s16, bf, c0, c1);
    bop[3] = dequant_slice<TT, BITS, FAST, 3>(wcur, sf, s16, bf, c0, c1);
    // Refill: weights of step t + GX_PF into this slot; after a (scale,
    // bias) slot's last step, its words of GX_UNROLL steps later.
    gx_wload<BITS>(src.wr, src.wl, t + GX_PF < cx.T ? src.woff(wpos) : src.wlast, wcur);
    wpos.step(cx.units);
    if (I == QS - 1) {
      gx_sbload<QS, GSQ>(src.sr, src.br, src.sl, t + 1 - QS + GX_UNROLL < cx.T ? src.soff(spos) : src.slast,
                         ring.s[q], ring.b[q]);
      spos.skip(QS, cx.units);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int mb = 0; mb < MBL; ++mb) {
        if constexpr (!kEarly) a[i][mb] = *reinterpret_cast<const u32x4*>(cx.xs + cx.aoff[i] + ub + mb * 4096);
        acc[mb] = Mfma16<TT>::run(a[i][mb], bop[i], acc[mb]);
      }
    if (cur.u == cx.units - 1) {  // slab done (uniform)
      if (cur.j < cx.my_slabs) {
        // Rows of the pass and columns inside n store; the others take an
        // offset past the buffer (rows without output: 2^31 plus the
        // column's bytes, still below 2^32), which drops the store.
        const int col = cx.col0 + 16 * GX_WAVES * cur.j;
        const bool colok = col < cx.n;
#pragma unroll
        for (int mb = 0; mb < MBL; ++mb) {
          // Rows 16 mb + 4 g + i of the pass, read from LDS here rather than
          // held in registers through the stream.
          const u32x4 o = *reinterpret_cast<const u32x4*>(cx.orow + 16 * mb + 4 * cx.g);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t off = colok ? o[i] + (uint32_t)col * 2u : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b16(TT::from_f32(acc[mb][i]), cx.yr, off, 0, 0);
          }
        }
      }
#pragma unroll
      for (int mb = 0; mb < MBL; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    cur.step(cx.units);
  }
}

// A run of groups with MBL 16-row blocks, each group dequantized the fast way
// when its (scale, bias) loads allow it.
template <typename TT, int BITS, int MB, int MBL, int QS, int GSQ>
__device__ __forceinline__ void gx_groups(const GxSrc& src, GxRing<BITS, QS, GSQ>& ring, GxPos wpos, GxPos spos,
                                          const GxCtx& cx) {
  f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  GxPos cur{0, 0};
  for (int t0 = 0; t0 < cx.T; t0 += GX_UNROLL) {
    // One decision per group: every (scale, bias) load the group reads.
    FastQuick fq;
    fast_quick_init(fq);
#pragma unroll
    for (int q = 0; q < GxRing<BITS, QS, GSQ>::kSb; ++q) gx_fast_add<TT, QS>(fq, ring.s[q], ring.b[q], cx.g);
    if (__builtin_amdgcn_ballot_w64(!fast_quick_ok<TT>(fq)) == 0ull)
      gx_group<TT, BITS, MB, MBL, true, QS, GSQ>(src, ring, wpos, spos, cur, t0, acc, cx);
    else
      gx_group<TT, BITS, MB, MBL, false, QS, GSQ>(src, ring, wpos, spos, cur, t0, acc, cx);
  }
}

// The pass's stream: the code for its number of 16-row blocks (only the
// blocks that hold rows of the pass are read and multiplied).
template <typename TT, int BITS, int MB, int QS, int GSQ>
__device__ __forceinline__ void gx_stream(const GxSrc& src, GxRing<BITS, QS, GSQ>& ring, GxPos wpos, GxPos spos,
                                          const GxCtx& cx) {
  if constexpr (MB >= 4)
    if (cx.mbl >= 3) {
      if (cx.mbl == 4) return gx_groups<TT, BITS, MB, 4, QS, GSQ>(src, ring, wpos, spos, cx);
      return gx_groups<TT, BITS, MB, 3, QS, GSQ>(src, ring, wpos, spos, cx);
    }
  if constexpr (MB >= 2)
    if (cx.mbl == 2) return gx_groups<TT, BITS, MB, 2, QS, GSQ>(src, ring, wpos, spos, cx);
  gx_groups<TT, BITS, MB, 1, QS, GSQ>(src, ring, wpos, spos, cx);
}

// First index i of the ascending a[0, n) with a[i] >= key (n if none), by one
// wave: each round splits the candidate range into 64 sub-ranges and counts
// the ones that end below key (a prefix, since a ascends) -- two rounds of
// loads for n <= 4096 instead of a serial bisection.
__device__ __forceinline__ int wave_lower_bound(const uint32_t* __restrict__ a, int n, uint32_t key, int lane) {
  int lo = 0, len = n;
  while (len > 1) {  // uniform
    const int step = (len + 63) / 64;
    const int last = lo + (lane + 1) * step - 1;  // last element of sub-range `lane`
    const bool below = last < lo + len && a[last] < key;
    const int c = __popcll(__ballot(below));
    lo += c * step;
    len = min(step, len - c * step);
  }
  if (len == 1 && a[lo] < key) ++lo;
  return lo;
}

// XOR key of row r (0..15) in the activation layout: the row's 2-bit halves
// swapped.  With the row itself as the key, lanes p, p+4, ..., p+60 (rows
// p, p+4, p+8, p+12 of the four chunk groups) meet in 4 slots, and
// SQ_LDS_BANK_CONFLICT counted 4 cycles per 16-byte operand read; with the
// swapped key it counts none.
__device__ __forceinline__ int gx_key(int r) { return ((r & 3) << 2) | (r >> 2); }

__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename TT, int BITS, int MB, int QS, int GSQ>
__global__ __launch_bounds__(GX_THREADS) void gather_expert_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, int x_rows,
    const uint32_t* __restrict__ lhs, const uint32_t* __restrict__ rhs, int n_rows,
    uint16_t* __restrict__ y, int n, int k, int gs_shift, int sorted, int nc,
    unsigned int* __restrict__ status) {
  static_assert(BITS == 4 || BITS == 8, "4- and 8-bit");
  constexpr int R = 16 * MB;
  __shared__ GxShared sh;
  extern __shared__ __attribute__((aligned(16))) unsigned char xs[];  // R x K activations
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const uint32_t e = blockIdx.y;
  const int c0 = blockIdx.x * nc;
  const int ncols = min(nc, n - c0);
  const int chunks = k >> 5;
  const int units = chunks >> 2;  // k % 128 == 0
  const int G = k >> gs_shift;
  const uint32_t row_bytes = (uint32_t)k * BITS / 8, grow_bytes = (uint32_t)G * 2u;
  const uint16_t* se = scales + (size_t)e * n * G;
  const uint16_t* be = biases + (size_t)e * n * G;

  // 0. Index validation, spread over the grid: workgroup b checks rows
  //    b * GX_THREADS + tid (+ multiples of the grid's threads).  A row with
  //    an expert index past the experts or an activation index past X is
  //    zeroed here (no workgroup stores it: no expert matches the first, the
  //    second's expert skips it) and counted, as is every descent of a
  //    sorted routing.  The first row's indices are loaded now and checked
  //    when the workgroup is done, so the loads never wait.
  const int ck_stride = gridDim.x * gridDim.y * GX_THREADS;
  const int ck_r0 = (blockIdx.y * gridDim.x + blockIdx.x) * GX_THREADS + tid;
  uint32_t ck_re = 0u, ck_le = 0u, ck_next = 0xffffffffu;
  if (ck_r0 < n_rows) {
    ck_re = rhs[ck_r0];
    ck_le = lhs ? lhs[ck_r0] : 0u;
    if (sorted && ck_r0 + 1 < n_rows) ck_next = rhs[ck_r0 + 1];
  }
  auto check_rows = [&]() {
    for (int r = ck_r0; r < n_rows; r += ck_stride) {
      uint32_t re = ck_re, le = ck_le, nx = ck_next;
      if (r != ck_r0) {
        re = rhs[r];
        le = lhs ? lhs[r] : 0u;
        nx = sorted && r + 1 < n_rows ? rhs[r + 1] : 0xffffffffu;
      }
      const bool bad = re >= gridDim.y || (lhs && le >= (uint32_t)x_rows);
      if (bad)
        for (int j = 0; j < n; ++j) y[(size_t)r * n + j] = 0;
      if (bad || (sorted && re > nx)) atomicAdd(status, 1u);
    }
  };

  // 1. Where this wave's weight stream reads (16-column slabs wave,
  //    wave + 8, ... of the chunk).
  const int nslab = (ncols + 15) >> 4;
  const int my_slabs = nslab > wave ? (nslab - wave + GX_WAVES - 1) / GX_WAVES : 0;
  const int T = my_slabs * units;  // steps of this wave
  GxSrc src;
  src.wr = __builtin_amdgcn_make_buffer_rsrc((void*)(w + (size_t)e * n * (row_bytes / 4)), 0,
                                             (int)((uint32_t)n * row_bytes), 0x00020000);
  src.sr = __builtin_amdgcn_make_buffer_rsrc((void*)se, 0, (int)((uint32_t)n * grow_bytes), 0x00020000);
  src.br = __builtin_amdgcn_make_buffer_rsrc((void*)be, 0, (int)((uint32_t)n * grow_bytes), 0x00020000);
  const int col0 = c0 + 16 * wave + nl;  // columns past n read past the buffers: zeros, never stored
  src.wl = (uint32_t)col0 * row_bytes + (uint32_t)g * (4u * BITS);
  src.sl = (uint32_t)col0 * grow_bytes + (QS == 1 ? (((uint32_t)g * 32u) >> gs_shift) * 2u : 0u);
  src.wslab = 16u * GX_WAVES * row_bytes;
  src.sslab = 16u * GX_WAVES * grow_bytes;
  src.wunit = 16u * BITS;               // 4 chunks of 4 * BITS bytes
  src.sunit = (256u >> gs_shift);       // 128 / gs groups of 2 bytes
  {
    const int tl = T > 0 ? T - 1 : 0;     // the last step (a wave without slabs re-reads step 0)
    const GxPos last{tl % units, tl / units};
    const GxPos lastq{last.u / QS * QS, last.j};
    src.wlast = src.woff(last);
    src.slast = src.soff(lastq);
  }
  GxRing<BITS, QS, GSQ> ring;
  GxPos wpos, spos;

  // 2. Rows routed to e, on a memory system not yet busy with this
  //    workgroup's weights (the routing, the activation rows and their
  //    loads are three dependent round trips).
  const int nblk = (n_rows + 63) >> 6;
  if (sorted) {
    if (n_rows <= GX_COUNT_ROWS) {
      // [lo, lo + total): rows below e and rows at e of the ascending rhs,
      // counted over every row in one round of loads.
      uint32_t v[GX_COUNT_ROWS / GX_THREADS];
#pragma unroll
      for (int j = 0; j < GX_COUNT_ROWS / GX_THREADS; ++j) {
        const int r = tid + j * GX_THREADS;
        v[j] = r < n_rows ? rhs[r] : 0xffffffffu;
      }
      int lt = 0, le = 0;
#pragma unroll
      for (int j = 0; j < GX_COUNT_ROWS / GX_THREADS; ++j) {
        lt += v[j] < e ? 1 : 0;
        le += v[j] <= e ? 1 : 0;
      }
      lt = wave_isum(lt);
      le = wave_isum(le);
      if (lane == 0) {
        sh.cnt[2 * wave] = lt;
        sh.cnt[2 * wave + 1] = le;
      }
      __syncthreads();
      if (tid == 0) {
        int a = 0, b = 0;
        for (int i = 0; i < GX_WAVES; ++i) {
          a += sh.cnt[2 * i];
          b += sh.cnt[2 * i + 1];
        }
        sh.lo = a;
        sh.total = b - a;
      }
    } else {
      // Equal range of e by two wave-parallel searches at once.
      if (wave < 2) {
        const int b = wave_lower_bound(rhs, n_rows, e + (uint32_t)wave, lane);
        if (lane == 0) sh.cnt[wave] = b;
      }
      __syncthreads();
      if (tid == 0) {
        sh.lo = sh.cnt[0];
        sh.total = sh.cnt[1] - sh.cnt[0];
      }
    }
  } else {
    // The first GX_KEEP blocks of each wave in one round of loads, their
    // match masks kept in LDS for the placement below, which then needs no
    // second load of rhs (kept in registers through the stream, they cost
    // the sorted routing 0.2-0.7 us); further blocks (past GX_KEEP * 512
    // rows) one at a time.
    uint32_t ev[GX_KEEP];
#pragma unroll
    for (int j = 0; j < GX_KEEP; ++j) {
      const int r = ((wave + GX_WAVES * j) << 6) + lane;
      ev[j] = r < n_rows ? rhs[r] : 0xffffffffu;
    }
#pragma unroll
    for (int j = 0; j < GX_KEEP; ++j) {
      const unsigned long long mk = __ballot(ev[j] == e);
      const int b = wave + GX_WAVES * j;
      if (lane == 0) {
        sh.keep[wave][j] = mk;
        if (b < nblk) sh.cnt[b] = __popcll(mk);
      }
    }
    for (int b = wave + GX_WAVES * GX_KEEP; b < nblk; b += GX_WAVES) {
      const int r = (b << 6) + lane;
      const unsigned long long mask = __ballot(r < n_rows && rhs[r] == e);
      if (lane == 0) sh.cnt[b] = __popcll(mask);
    }
    __syncthreads();
    if (tid == 0) {  // exclusive prefix over the blocks
      int run_ = 0;
      for (int b = 0; b < nblk; ++b) {
        const int c = sh.cnt[b];
        sh.cnt[b] = run_;
        run_ += c;
      }
      sh.total = run_;
      sh.lo = 0;
    }
  }

  __syncthreads();
  const int total = sh.total;
  if (total == 0) {  // uniform
    check_rows();
    return;
  }

  // LDS offsets of this lane's A pieces: 16-byte piece i of chunk 4u + g of
  // row nl of a block is slot (4g + i) ^ key(nl) of the row (unit u, block mb
  // at (u * MB + mb) * 4096 bytes).
  GxCtx cx;
  cx.T = T;
  cx.units = units;
  cx.my_slabs = my_slabs;
  cx.g = g;
  cx.sel = gx_sb_sel<TT>(g);
#pragma unroll
  for (int i = 0; i < 4; ++i) cx.aoff[i] = (uint32_t)nl * 256u + (uint32_t)(((4 * g + i) ^ gx_key(nl)) * 16);
  cx.xs = xs;
  cx.orow = sh.orow;
  cx.col0 = col0;
  cx.n = n;
  cx.yr = __builtin_amdgcn_make_buffer_rsrc((void*)y, 0, (int)((uint32_t)n_rows * (uint32_t)n * 2u), 0x00020000);

  for (int p0 = 0; p0 < total; p0 += R) {
    // 3. The pass's rows and activation rows.
    if (tid < R) sh.rows[tid] = -1;
    __syncthreads();
    if (sorted) {
      if (tid < R && p0 + tid < total) sh.rows[tid] = sh.lo + p0 + tid;
    } else {
      // Block b's matches, ranked within the expert: its count prefix plus
      // the matches below this lane.
      auto place = [&](int b, unsigned long long mask) {
        const int base = sh.cnt[b];
        const int next = b + 1 < nblk ? sh.cnt[b + 1] : total;
        if (next <= p0 || base >= p0 + R) return;  // uniform per wave
        const int r = (b << 6) + lane;
        const bool match = (mask >> lane) & 1ull;
        const int rank = base + __popcll(mask & ((1ull << lane) - 1ull));
        if (match && rank >= p0 && rank < p0 + R) sh.rows[rank - p0] = r;
      };
#pragma unroll
      for (int j = 0; j < GX_KEEP; ++j) {
        const int b = wave + GX_WAVES * j;
        if (b < nblk) place(b, sh.keep[wave][j]);
      }
      for (int b = wave + GX_WAVES * GX_KEEP; b < nblk; b += GX_WAVES) {
        const int r = (b << 6) + lane;
        place(b, __ballot(r < n_rows && rhs[r] == e));
      }
    }
    __syncthreads();
    if (tid < R) {
      const int r = sh.rows[tid];
      int xi = -1;
      if (r >= 0) {
        const uint32_t v = lhs ? lhs[r] : (uint32_t)r;
        if (v < (uint32_t)x_rows) xi = (int)v;
      }
      sh.xrow[tid] = xi;
    }
    __syncthreads();

    // 4. Activation rows into LDS in the dequantizer's slot order: every
    //    16-byte item of the pass (at most GX_XITEMS per thread) requested at
    //    once, then the first weight steps (so the activations do not queue
    //    behind them), then the LDS writes.  Only the pass's rows are
    //    staged: the other rows of its 16-row blocks keep stale LDS bytes,
    //    which reach only their own output rows (MFMA rows are independent),
    //    and those are not stored.
    const int kq = k >> 3;  // 16-byte items per row
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)x_rows * (uint32_t)k * 2u), 0x00020000);
    const int nst = min(R, total - p0) * kq;  // <= R * K / 8
    // Rounds of GX_XITEMS items per thread (one round when that covers
    // R * K / 8); the bound is uniform, and nst > 0, so every thread runs the
    // first round and issues the weight steps in it.
    for (int base = 0; base < nst; base += GX_XITEMS * GX_THREADS) {
      int id0 = base + tid;
      // Opaque per pass: the items' indices and offsets are recomputed here
      // instead of being hoisted out of the pass loop and held (or spilled)
      // through the stream.
      __asm__ __volatile__("" : "+v"(id0));
      // Item id = id0 + h * GX_THREADS is row id / kq, 16-byte piece id % kq;
      // both advance by fixed amounts per h (one division, not one per item).
      const int di = GX_THREADS / kq, dq = GX_THREADS - di * kq;
      int ii[GX_XITEMS], qq[GX_XITEMS];
      ii[0] = id0 / kq;
      qq[0] = id0 - ii[0] * kq;
#pragma unroll
      for (int h = 1; h < GX_XITEMS; ++h) {
        const int q1 = qq[h - 1] + dq;
        const bool wrap = q1 >= kq;
        qq[h] = wrap ? q1 - kq : q1;
        ii[h] = ii[h - 1] + di + (wrap ? 1 : 0);
      }
      // Every item is requested (no branch, so the count of loads in
      // flight stays exact): items past the pass or of an invalid row take
      // an offset past the buffer and read zeros.
      u32x4 v[GX_XITEMS];
#pragma unroll
      for (int h = 0; h < GX_XITEMS; ++h) {
        const int id = id0 + h * GX_THREADS;
        const int xi = id < nst ? sh.xrow[min(ii[h], R - 1)] : -1;
        const uint32_t off = xi >= 0 ? ((uint32_t)xi * (uint32_t)k + (uint32_t)qq[h] * 8u) * 2u : 0x80000000u;
        v[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
      if (base == 0) gx_fill<BITS, QS, GSQ>(src, ring, T, units, wpos, spos);
#pragma unroll
      for (int h = 0; h < GX_XITEMS; ++h) {
        const int id = id0 + h * GX_THREADS;
        if (id < nst) {
          const int i = ii[h], q = qq[h];
          const int r16 = i & 15;
          const uint32_t off = (uint32_t)((q >> 4) * MB + (i >> 4)) * 4096u + (uint32_t)r16 * 256u +
                               (uint32_t)(((q & 15) ^ gx_key(r16)) * 16);
          *reinterpret_cast<u32x4*>(xs + off) = interleave_x<BITS>(v[h]);
        }
      }
    }
    // The pass's output rows, as byte offsets into Y (2^31: none).
    if (tid < R)
      sh.orow[tid] = sh.rows[tid] >= 0 && sh.xrow[tid] >= 0 ? (uint32_t)sh.rows[tid] * (uint32_t)n * 2u : 0x80000000u;
    __syncthreads();

    // 5. Stream the weights of this wave's slabs (again for every further
    //    pass).
    cx.mbl = (min(R, total - p0) + 15) >> 4;
    if (T > 0) gx_stream<TT, BITS, MB, QS, GSQ>(src, ring, wpos, spos, cx);
    __syncthreads();  // LDS rows / activations are rewritten by the next pass
  }
  check_rows();
}

template <typename TT, int BITS, int MB, int QS, int GSQ>
hipError_t launch_q(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                    const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                    int gs_shift, int n_chunks, int nc, unsigned int* status) {
  static const hipError_t attr = [] {
    const void* fn = reinterpret_cast<const void*>(&gather_expert_kernel<TT, BITS, MB, QS, GSQ>);
    hipFuncAttributes fa;
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(160 * 1024 - fa.sharedSizeBytes));
  }();
  if (attr != hipSuccess) return attr;
  const size_t lds = (size_t)16 * MB * k * 2;
  hipLaunchKernelGGL((gather_expert_kernel<TT, BITS, MB, QS, GSQ>), dim3((unsigned)n_chunks, (unsigned)n_experts),
                     dim3(GX_THREADS), lds, s, q.w, static_cast<const uint16_t*>(q.scales),
                     static_cast<const uint16_t*>(q.biases), static_cast<const uint16_t*>(x), x_rows, lhs,
                     rhs, n_rows, static_cast<uint16_t*>(y), n, k, gs_shift, (int)sorted, nc, status);
  return hipGetLastError();
}

// Scale / bias quads: 4 steps per 16-byte load (gs 64) or 8-byte load (gs
// 128) when a slab's units divide by 4, else 2 steps per 8-byte load (gs 64),
// else per-step 2-byte loads.  Alignment: row starts are multiples of the
// vector (G a multiple of its groups) and the base pointers aligned to it.
template <typename TT, int BITS, int MB>
hipError_t launch_mb(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                     const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                     int gs_shift, int n_chunks, int nc, unsigned int* status) {
  const int G = k / q.gs, units = k / 128;
  const uintptr_t al = reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases);
  // Buffer offsets of one expert's tables and of Y stay inside 31 bits.
  if ((uint64_t)n * k * BITS / 8 >= (1ull << 31) || (uint64_t)n * G * 2 >= (1ull << 31) ||
      (uint64_t)n_rows * n * 2 >= (1ull << 31) || (uint64_t)x_rows * k * 2 >= (1ull << 31))
    return hipErrorInvalidValue;
  static const int forced = env_int("CPQ_GATHER_QS", 0);
#define CPQ_GXQ(QS, GSQ)                                                                                  \
  return launch_q<TT, BITS, MB, QS, GSQ>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted,   \
                                         gs_shift, n_chunks, nc, status)
  // Each expert's tables start (n G entries apart) aligned to the vector too.
  const long eb = (long)n * G * 2;
  if (forced != 1) {
    if (q.gs == 64 && units % 4 == 0 && al % 16 == 0 && eb % 16 == 0 && forced != 2) CPQ_GXQ(4, 64);
    if (q.gs == 64 && units % 2 == 0 && al % 8 == 0 && eb % 8 == 0) CPQ_GXQ(2, 64);
    if (q.gs == 128 && units % 4 == 0 && al % 8 == 0 && eb % 8 == 0) CPQ_GXQ(4, 128);
  }
  CPQ_GXQ(1, 64);
#undef CPQ_GXQ
}

template <typename TT, int BITS>
hipError_t launch_t(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                    const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                    int cu_count, unsigned int* status) {
  int gs_shift = 0;
  while ((1 << gs_shift) < q.gs) ++gs_shift;
  // Column chunks (whole multiples of 8 slabs = 128 columns): the count that
  // minimises rounds-of-workgroups x work-per-workgroup over the CUs.
  const int slabs128 = (n + 127) / 128;
  int best = 1;
  long best_cost = -1;
  for (int c = 1; c <= slabs128; ++c) {
    const long rounds = ((long)c * n_experts + cu_count - 1) / cu_count;
    const long cost = rounds * ((slabs128 + c - 1) / c);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = c;
    }
  }
  const int nc = (slabs128 + best - 1) / best * 128;
  const int n_chunks = (n + nc - 1) / nc;
  if ((size_t)64 * k * 2 <= (size_t)GX_XBYTES)
    return launch_mb<TT, BITS, 4>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, gs_shift,
                                  n_chunks, nc, status);
  if ((size_t)32 * k * 2 <= (size_t)GX_XBYTES)
    return launch_mb<TT, BITS, 2>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, gs_shift,
                                  n_chunks, nc, status);
  return launch_mb<TT, BITS, 1>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, gs_shift,
                                n_chunks, nc, status);
}

}  // namespace

bool gather_expert_supported(int bits, int x_rows, int n_rows, int n, int k) {
  // k % 128: whole units per staged row; X, one expert's weights and Y
  // within the 31-bit buffer offsets.
  return (bits == 4 || bits == 8) && k % 128 == 0 && n_rows <= 64 * GX_MAXBLK &&
         (uint64_t)x_rows * k * 2 < (1ull << 31) &&
         (size_t)16 * k * 2 <= (size_t)GX_XBYTES && (uint64_t)n * k * bits / 8 < (1ull << 31) &&
         (uint64_t)n_rows * n * 2 < (1ull << 31);
}

hipError_t launch_gather_expert(hipStream_t s, const QuantArgs& q, const void* x, int x_rows,
                                const uint32_t* lhs, const uint32_t* rhs, int n_rows, void* y,
                                int n_experts, int n, int k, bool sorted, int cu_count,
                                unsigned int* status) {
#define CPQ_GX(TT)                                                                                        \
  switch (q.bits) {                                                                                       \
    case 4: return launch_t<TT, 4>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, cu_count, status); \
    case 8: return launch_t<TT, 8>(s, q, x, x_rows, lhs, rhs, n_rows, y, n_experts, n, k, sorted, cu_count, status); \
    default: return hipErrorInvalidValue;                                                                 \
  }
  if (q.dtype == CPQ_DTYPE_BF16) { CPQ_GX(BF16) }
  if (q.dtype == CPQ_DTYPE_F16) { CPQ_GX(F16) }
#undef CPQ_GX
  return hipErrorInvalidValue;
}

}  // namespace cpq
