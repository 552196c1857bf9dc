// Prefill quantized GEMM for gfx950, two waves per SIMD (4-bit weights).
//
// Reference op: affine_qmm_t / qmm_t_impl (kernels-mlx/mlx/backend/metal/
// kernels/quantized.h:1087-1213, 1713-1784), dispatched by
// crates/cider-press-kernels/src/kernels/qmm.rs:66-220.  Numerics as every
// other path here: each weight is dequantized to T (RNE of fmaf(s, q, b)),
// products accumulate in fp32 on the matrix cores, the output is rounded to
// T once.
//
// Why this shape.  Measured on MI355X, one wave per SIMD issues an
// instruction only every ~5.5 cycles, so a single wave cannot both feed the
// matrix pipe (one v_mfma_f32_32x32x16 per 32 cycles) and do the ~4.5 VALU
// instructions of dequantization each MFMA needs at a 128-row tile; two
// waves per SIMD hide up to ~6 VALU instructions per MFMA.  Two waves per
// SIMD leave each wave 256 registers, so a wave holds a 128 x 64 accumulator
// (128 fp32 per lane) and the workgroup splits K between waves.
//
// Workgroup: 512 threads (8 waves), tile 128 (M) x 128 (N), K range
// [kb0, kb0 + K/split) in stages of 128.  Wave w: K quarter kq = w & 3 (k
// [32 kq, 32 kq + 32) of every stage), N half nh = w >> 2 (columns
// [64 nh, 64 nh + 64)).
//   A (activations): a 3-slot LDS ring, 32 KiB per stage, filled by
//      buffer_load_dwordx4 ... lds two stages ahead; each copy instruction
//      moves 4 rows x 256 B; 16-B chunks are XOR-swizzled by row so the MFMA
//      fragment reads (ds_read_b128) are conflict-free.
//   W (packed weights): a 3-slot LDS ring, 8 KiB per stage (128 columns x
//      64 B), filled by the same DMA three stages ahead.  A column's 16-B
//      chunk q (= K quarter q of the stage) sits at position q ^ ((c >> 2) & 3)
//      of its 64-B row, so the waves' 8-byte reads hit every bank pair twice.
//      W's slot for stage s+3 is the one of stage s: a wave dequantizes a
//      stage's weights during the stage before, so by stage s nobody reads it.
//   Constants: raw (scale, bias) 16-bit pairs of the tile's columns for every
//      group of the K range, staged once; the workgroup votes on the fast
//      dequantization (fastpath.hpp) from the same loads.
//   Per stage a wave runs 16 MFMAs (4 row blocks x 2 column blocks x 2 k
//   steps) on operands dequantized during the previous stage, and between
//   them dequantizes the next stage's 4 B operands (8 weights per lane each).
//   The MFMA k order inside the wave's 32-k slice is permuted so that lane
//   half h needs k units 2h, 2h+1: one 8-byte LDS read per column block.
//   Epilogue: the four K-quarter partials of each N half are summed through
//   LDS in two row halves; with split > 1 the workgroups of a tile exchange
//   fp32 partial tiles through scratch and the last to arrive adds them in
//   k-part order (deterministic) and resets the tile's arrival counter.
// MFMA 32x32x16 layout: A[m][k] lane m%32 + 32(k/8), element k%8; B[k][n]
// lane n%32 + 32(k/8), element k%8; D[m][n] lane n + 32((m/4)%2), element
// 4(m/8) + m%4.
#include <algorithm>

#include <type_traits>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int DBM = 128, DBN = 128, DBK = 128;
constexpr int DNS = 3;                          // ring slots (A and W)
constexpr int DASLOT = DBM * DBK * 2;           // 32 KiB of activations per stage
constexpr int DWSLOT = DBN * DBK / 2;           // 8 KiB of 4-bit weights per stage
constexpr int DWBASE = DNS * DASLOT;            // W ring after the A ring
constexpr int DRING = DNS * (DASLOT + DWSLOT);  // 120 KiB; constants follow
constexpr int DMAXB = 2;                        // 8-group constant blocks per thread: K range / gs <= 64
constexpr int DEPI = 64 + 4;                    // epilogue floats per lane (padded)
constexpr int DEPI_BYTES = 8 * 64 * DEPI * 4;   // 139264
constexpr int DLDS_MAX = 160 * 1024 - 256;      // dynamic LDS budget next to the vote words
constexpr int DPART = DBM * DBN;                // floats per partial tile
// Split-K words at the head of the scratch (64 KiB): per tile at [t] the
// arrivals (low 8 bits) and, bit 8 + kk, k-part kk parked through its XCD's
// L2; per (tile, k-part) the XCD id + 1 of the workgroup computing it at
// [kDmaXccOffset + t*split + kk].  All are zero between launches.
constexpr int kDmaMaxTiles = 4096;
constexpr int kDmaXccOffset = 10240;
constexpr int kDmaMaxParts = 6144;  // tiles * split

struct DmaGeom {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xoff[4];   // A copy source of this lane, copy j (stage 0 of the K range)
  uint32_t woff;      // W copy source of this lane (stage 0)
  uint32_t a_off[2];  // A fragment of k step t, row block 0, within a slot
  uint32_t w_off[2];  // 8-byte weight read of column block cb within a slot
  uint32_t c_off;     // constants of this lane's column (block 0, group 0)
  unsigned char* smem;
  int wave, kq, gs_shift, S;
};

template <typename TT>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (Sig16<TT>::bf16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// This wave's 4 activation copies of stage st into the A slot at byte
// offset `slot`.
__device__ __forceinline__ void dma_a(const DmaGeom& g, int st, int slot) {
  unsigned char* a = g.smem + slot;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(g.xr, (__attribute__((address_space(3))) void*)(a + (g.wave * 4 + j) * 1024),
                                             16, g.xoff[j], st * (DBK * 2), 0, 0);
}

// This wave's weight copy of stage st (1 KiB) into the W slot at byte
// offset `slot` from the W ring.
__device__ __forceinline__ void dma_w(const DmaGeom& g, int st, int slot) {
  unsigned char* w = g.smem + DWBASE + slot;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(g.wr, (__attribute__((address_space(3))) void*)(w + g.wave * 1024), 16,
                                           g.woff, st * (DBK / 2), 0, 0);
}

// Per-column dequantization constants of one group: f32 scale, and either
// c0 = b - 1024 s and c1 = b - 64 s (fast) or the bias (generic).
struct Cst {
  float s, c0, c1;
};

template <typename TT, bool FAST>
__device__ __forceinline__ Cst make_cst(uint32_t sb) {
  Cst c;
  c.s = TT::to_f32((uint16_t)(sb & 0xffffu));
  const float b = TT::to_f32((uint16_t)(sb >> 16));
  if constexpr (FAST) {
    c.c0 = fmaf(-1024.f, c.s, b);
    c.c1 = fmaf(960.f, c.s, c.c0);
  } else {
    c.c0 = b;
    c.c1 = 0.f;
  }
  return c;
}

// 8 nibbles of one word (k order) -> MFMA B operand in k order.  Fast path:
// v_and_or drops e_even into the mantissa of f16 1024 (0x6400) and e_odd,
// left in place as 16e, into f16 64 (0x5400, giving 64 + e); one
// v_fma_mix_f32 each computes s(1024 + e) + c0 or s(64 + e) + c1, i.e.
// fmaf(s, e, b) exactly when c0, c1 are exact (the workgroup vote).
template <typename TT, bool FAST>
__device__ __forceinline__ u32x4 dequant_word(uint32_t word, const Cst& c) {
  if constexpr (FAST) {
    const uint32_t w8 = word >> 8;
    const uint32_t p0 = and_or(word, 0x000F000Fu, 0x64006400u);  // (1024 + e0, 1024 + e4)
    const uint32_t p1 = and_or(word, 0x00F000F0u, 0x54005400u);  // (64 + e1, 64 + e5)
    const uint32_t p2 = and_or(w8, 0x000F000Fu, 0x64006400u);    // (1024 + e2, 1024 + e6)
    const uint32_t p3 = and_or(w8, 0x00F000F0u, 0x54005400u);    // (64 + e3, 64 + e7)
    return u32x4{TT::pack2(fmaf(c.s, f16lo(p0), c.c0), fmaf(c.s, f16lo(p1), c.c1)),
                 TT::pack2(fmaf(c.s, f16lo(p2), c.c0), fmaf(c.s, f16lo(p3), c.c1)),
                 TT::pack2(fmaf(c.s, f16hi(p0), c.c0), fmaf(c.s, f16hi(p1), c.c1)),
                 TT::pack2(fmaf(c.s, f16hi(p2), c.c0), fmaf(c.s, f16hi(p3), c.c1))};
  } else {
    const uint32_t wd[1] = {word};
    return dequant_slice_nat<TT, 4, false, 0>(wd, c.s, c.s * 0.0625f, c.c0, 0.f, 0.f);
  }
}

// Weight words and raw constants of stage st for this wave (2 column blocks).
struct StageW {
  u32x2 w[2];      // words for k steps 0, 1 of column block cb
  uint32_t sb[2];  // raw (scale, bias) of column block cb
};

__device__ __forceinline__ StageW read_stage_w(const DmaGeom& g, int st, int wslot) {
  StageW r;
  const unsigned char* w = g.smem + DWBASE + wslot;
  const int grp = (st * DBK + 32 * g.kq) >> g.gs_shift;
  const unsigned char* cs = g.smem + DRING + g.c_off + grp * (DBN * 4);
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    r.w[cb] = *reinterpret_cast<const u32x2*>(w + g.w_off[cb]);
    r.sb[cb] = *reinterpret_cast<const uint32_t*>(cs + cb * 128);
  }
  return r;
}

template <typename TT, bool FAST>
__device__ __forceinline__ void dequant_stage(const StageW& sw, u32x4 (&b)[2][2]) {
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const Cst c = make_cst<TT, FAST>(sw.sb[cb]);
#pragma unroll
    for (int t = 0; t < 2; ++t) b[cb][t] = dequant_word<TT, FAST>(sw.w[cb][t], c);
  }
}

// Wait for all but N vector-memory loads of this wave and for its LDS accesses.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// Ring slots rotate through 3 byte offsets; `ra` is stage s's A slot.
__device__ __forceinline__ int next_slot(int ra) { return ra == 2 * DASLOT ? 0 : ra + DASLOT; }
__device__ __forceinline__ int prev_slot(int ra) { return ra == 0 ? 2 * DASLOT : ra - DASLOT; }

// Stage kinds: copies still to issue near the end of the K range.
enum { ST_MAIN = 0, ST_LAST3 = 1, ST_LAST2 = 2, ST_LAST1 = 3 };

// One stage, skewed by half a stage: after stage s's barrier the wave first
// runs stage s-1's second k step (its A fragments and B operands are in
// registers already), which keeps the matrix cores busy while stage s's A
// fragments arrive from LDS, then stage s's first k step; between them it
// dequantizes stage s+1's B operands.
//   acur <- A(s) fragments; aprev holds A(s-1) (k step 1 still to run);
//   bcur holds B(s) (dequantized during stage s-1); bprev holds B(s-1);
//   bprev is overwritten with B(s+1) once its k step 1 has been issued.
// Copies per stage and wave: A(s+2) x 4 then W(s+3) x 1 while those stages
// exist (the prologue issues W0, A0 x 4, W1, A1 x 4, W2; stage S-3 issues
// only A(S-1); the last two issue nothing).  So at the start of stage s "all
// but the younger copies" -- 5 for a main stage and for S-3, 4 for S-2,
// none for S-1 -- proves that A(s) and W(s+1) landed for this wave; the
// barrier extends that to every wave and frees the slots refilled next (A
// slot of stage s-1 and W slot of stage s, both read before this barrier).
template <typename TT, bool FAST, int KIND, bool PREV>
__device__ __forceinline__ void dma_stage(const DmaGeom& g, int s, int ra, u32x4 (&acur)[4][2],
                                          const u32x4 (&aprev)[4][2], const u32x4 (&bcur)[2][2],
                                          u32x4 (&bprev)[2][2], f32x16 (&acc)[4][2]) {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  if constexpr (KIND == ST_LAST1)
    wait_vm_lgkm<0>();
  else if constexpr (KIND == ST_LAST2)
    wait_vm_lgkm<4>();
  else
    wait_vm_lgkm<5>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  if constexpr (KIND == ST_MAIN || KIND == ST_LAST3) dma_a(g, s + 2, prev_slot(ra));
  if constexpr (KIND == ST_MAIN) dma_w(g, s + 3, ra >> 2);
  const unsigned char* aslot = g.smem + ra;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acur[i][t] = *reinterpret_cast<const u32x4*>(aslot + g.a_off[t] + i * 8192);
  StageW sw;
  if constexpr (KIND != ST_LAST1) sw = read_stage_w(g, s + 1, next_slot(ra) >> 2);
  if constexpr (PREV) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i][cb] = mfma32<TT>(aprev[i][1], bprev[cb][1], acc[i][cb]);
  }
  if constexpr (KIND != ST_LAST1) dequant_stage<TT, FAST>(sw, bprev);
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i][cb] = mfma32<TT>(acur[i][0], bcur[cb][0], acc[i][cb]);
}

// Stage S-1's second k step, after the loop.
template <typename TT>
__device__ __forceinline__ void dma_tail(const u32x4 (&alast)[4][2], const u32x4 (&blast)[2][2], f32x16 (&acc)[4][2]) {
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i][cb] = mfma32<TT>(alast[i][1], blast[cb][1], acc[i][cb]);
}

// S is even and at least 8: stage 0 (nothing before it), stages 1 .. S-5 in
// pairs, then S-4 (even), and the last three with their own copy counts.
// Even stages use (a0, b0) as current and (a1, b1) as previous; odd stages
// the other way round.
template <typename TT, bool FAST>
__device__ __forceinline__ void dma_loop(const DmaGeom& g, f32x16 (&acc)[4][2]) {
  // Stage 0's operands: W0 and the constants are visible (prologue barrier).
  u32x4 a0[4][2], a1[4][2], b0[2][2], b1[2][2];
  dequant_stage<TT, FAST>(read_stage_w(g, 0, 0), b0);
  int ra = 0;
  dma_stage<TT, FAST, ST_MAIN, false>(g, 0, ra, a0, a1, b0, b1, acc);
  ra = next_slot(ra);
  int s = 1;
  for (; s < g.S - 4; s += 2) {
    dma_stage<TT, FAST, ST_MAIN, true>(g, s, ra, a1, a0, b1, b0, acc);
    ra = next_slot(ra);
    dma_stage<TT, FAST, ST_MAIN, true>(g, s + 1, ra, a0, a1, b0, b1, acc);
    ra = next_slot(ra);
  }
  // s == S-3 here (S even): stages S-3 (odd), S-2 (even), S-1 (odd).
  dma_stage<TT, FAST, ST_LAST3, true>(g, s, ra, a1, a0, b1, b0, acc);
  ra = next_slot(ra);
  dma_stage<TT, FAST, ST_LAST2, true>(g, s + 1, ra, a0, a1, b0, b1, acc);
  ra = next_slot(ra);
  dma_stage<TT, FAST, ST_LAST1, true>(g, s + 2, ra, a1, a0, b1, b0, acc);
  dma_tail<TT>(a1, b1, acc);
}

template <typename TT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void qmm_dma_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int m, int n, int k, int gs_shift, int tiles_m,
    int tiles_n, int split, float* __restrict__ part, unsigned int* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = wave & 3, nh = wave >> 2;
  const int l32 = lane & 31, h = lane >> 5;

  // Workgroup order: each XCD (linear ids congruent mod 8) takes a
  // contiguous run of (tile, k-part) pairs, k-part fastest, then M tiles, so
  // the k-parts of a tile share one L2 and the run shares panels of X and W.
  const int nwg = tiles_m * tiles_n * split;
  int v = blockIdx.x;
  if ((nwg & 7) == 0) v = (v & 7) * (nwg >> 3) + (v >> 3);
  const int kh = v % split, t = v / split;
  const int mt = t % tiles_m, nt = t / tiles_m;
  const int row0 = mt * DBM, col0 = nt * DBN;
  const int KL = k / split, kb0 = kh * KL;
  const int G = k >> gs_shift, GL = KL >> gs_shift, gk0 = kb0 >> gs_shift;
  const uint32_t rowbytes = (uint32_t)k / 2u;

  DmaGeom g;
  g.smem = smem;
  g.wave = wave;
  g.kq = kq;
  g.gs_shift = gs_shift;
  g.S = KL / DBK;
  g.xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);
  g.wr = __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  // A copy block b = 4*wave + j holds rows 4b .. 4b+3; lane i lands at row
  // 4b + i/16, physical chunk i%16, which holds logical chunk (i%16)^(row%16).
  // Rows past M re-read row M-1 (never stored).
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int rr = (wave * 4 + j) * 4 + (lane >> 4);
    const int c = (lane & 15) ^ (rr & 15);
    const int grow = min(row0 + rr, m - 1);
    g.xoff[j] = ((uint32_t)grow * (uint32_t)k + (uint32_t)kb0 + (uint32_t)(c * 8)) * 2u;
  }
  // W copy: LDS chunk L = 64*wave + lane is column L/4, position L%4, which
  // holds the column's K quarter q = (L%4) ^ ((column >> 2) & 3).  Columns
  // past N read zeros through the descriptor's range check (never stored).
  {
    const int c = 16 * wave + (lane >> 2);
    const int q = (lane & 3) ^ ((c >> 2) & 3);
    g.woff = (uint32_t)(col0 + c) * rowbytes + (uint32_t)kb0 / 2u + (uint32_t)(16 * q);
  }
  // A fragment of lane (l32, h), k step t: row 32i + l32, the stage's
  // logical chunk 4kq + 2h + t (k units 2h, 2h+1 of the wave's slice).
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
    g.a_off[tt] = (uint32_t)(l32 * 256 + (((4 * kq + 2 * h + tt) ^ (l32 & 15)) * 16));
  // Weights of lane (l32, h), column block cb: column 64nh + 32cb + l32, its
  // K quarter kq, bytes 8h .. 8h+7 (words 2h, 2h+1 = k steps 0, 1).
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int c = 64 * nh + 32 * cb + l32;
    g.w_off[cb] = (uint32_t)(16 * (4 * c + (kq ^ ((c >> 2) & 3))) + 8 * h);
  }
  g.c_off = (uint32_t)(64 * nh + l32) * 4u;

  // 1. Scale / bias words of the tile's columns: thread (column tid % 128,
  //    part tid / 128) loads 8-group blocks part, part + 4 (16-B loads; G,
  //    the K-range start and the pointers are 16-B aligned).  Issued first,
  //    consumed once the stream copies are in flight.
  const int cc = tid & 127, part_ = tid >> 7;
  const int ccol = min(col0 + cc, n - 1);
  u32x4 sv[DMAXB], bv[DMAXB];
#pragma unroll
  for (int u = 0; u < DMAXB; ++u) {
    const int gb = part_ + 4 * u;
    if (8 * gb < GL) {
      const size_t off = (size_t)ccol * G + gk0 + 8 * gb;
      sv[u] = *reinterpret_cast<const u32x4*>(scales + off);
      bv[u] = *reinterpret_cast<const u32x4*>(biases + off);
    }
  }

  // 2. Stream copies of stage 0 (the vote below waits for them anyway).
  __builtin_amdgcn_sched_barrier(0);
  dma_w(g, 0, 0);
  dma_a(g, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  // With split K, publish the XCD this workgroup runs on (hardware register
  // XCC_ID; each XCD has its own L2): the parts of a tile on one XCD can
  // exchange their partial tiles through that L2.
  const uint32_t xcc1 = (__builtin_amdgcn_s_getreg(20 | (31 << 11)) & 0xfu) + 1u;
  if (split > 1 && tid == 0)
    __hip_atomic_store(&counters[kDmaXccOffset + t * split + kh], xcc1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // 3. Constants into LDS: (s | b << 16) at [group][column].  Each thread
  //    checks its groups (packed exponent check; the exact predicate only
  //    when that one is inconclusive); the workgroup votes below.
  uint32_t* cst = reinterpret_cast<uint32_t*>(smem + DRING);
  FastQuick fq;
  fast_quick_init(fq);
#pragma unroll
  for (int u = 0; u < DMAXB; ++u)
    if (8 * (part_ + 4 * u) < GL)
#pragma unroll
      for (int q = 0; q < 4; ++q) fast_quick_add<TT>(fq, sv[u][q], bv[u][q]);
  bool ok = fast_quick_ok<TT>(fq);
  if (!ok) {
    ok = true;
#pragma unroll
    for (int u = 0; u < DMAXB; ++u)
      if (8 * (part_ + 4 * u) < GL)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ok &= fast_ok_bits<TT>(sv[u][q] & 0xffffu, bv[u][q] & 0xffffu) &
                fast_ok_bits<TT>(sv[u][q] >> 16, bv[u][q] >> 16);
  }
#pragma unroll
  for (int u = 0; u < DMAXB; ++u) {
    const int gb = part_ + 4 * u;
    if (8 * gb < GL) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cst[(8 * gb + 2 * q) * DBN + cc] = (sv[u][q] & 0xffffu) | (bv[u][q] << 16);
        cst[(8 * gb + 2 * q + 1) * DBN + cc] = (sv[u][q] >> 16) | (bv[u][q] & 0xffff0000u);
      }
    }
  }
  // The remaining copies of the prologue, in the steady-state order (W0, A0
  // x 4, W1, A1 x 4, W2; S >= 8, so all exist).
  __builtin_amdgcn_sched_barrier(0);
  dma_w(g, 1, DWSLOT);
  dma_a(g, 1, DASLOT);
  dma_w(g, 2, 2 * DWSLOT);
  __builtin_amdgcn_sched_barrier(0);
  // Vote through one LDS word per wave.  Then wait for this wave's W0 (its
  // first copy; the 10 younger copies may still fly) and its constant
  // stores; the barrier makes every wave's W0, constants and vote visible.
  __shared__ uint32_t dma_vote[8];
  __shared__ uint32_t dma_flags[2];  // split-K: [0] arrival word, [1] this part parks through the L2
  const bool wave_ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
  if (lane == 0) dma_vote[wave] = wave_ok ? 1u : 0u;
  asm volatile("" ::: "memory");
  wait_vm_lgkm<10>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  uint32_t all = 1u;
#pragma unroll
  for (int i = 0; i < 8; ++i) all &= dma_vote[i];
  const bool fast = all != 0u;

  // 4. Stream K.
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][cb][e] = 0.f;
  if (fast)
    dma_loop<TT, true>(g, acc);
  else
    dma_loop<TT, false>(g, acc);

  // 5. Sum the four K quarters of each N half through LDS, in two row
  //    halves.  Round r: every wave parks row blocks 2r, 2r+1 (both column
  //    blocks: 64 floats per lane); wave (kq', nh) then adds, for lane L,
  //    the 16 floats of block (2r + kq'/2, kq'%2) over the four K quarters.
  // Split K: whether every other part of this tile runs on this XCD (their
  // published ids; one not yet published counts as elsewhere).  Read now,
  // used after the reduction below.
  if (split > 1 && tid == 0) {
    uint32_t local = 1u;
    for (int kk = 0; kk < split; ++kk)
      if (kk != kh)
        local &= __hip_atomic_load(&counters[kDmaXccOffset + t * split + kk], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == xcc1
                     ? 1u
                     : 0u;
    dma_flags[1] = local;
  }
  __syncthreads();  // every wave done with the rings (all copies landed: the last stage waited for them)
  float* ep = reinterpret_cast<float*>(smem);
  f32x16 res[2];
  // Specialised by the wave's K quarter: a wave parks only the three blocks
  // other waves add (its own block, slot kq, stays in registers) and reads
  // the other three quarters' slot kq; the sums keep K-quarter order.
  auto reduce = [&](auto KQ) {
    constexpr int KQC = decltype(KQ)::value;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float* mine = ep + (wave * 64 + lane) * DEPI;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          if (ii * 2 + cb == KQC) continue;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4*>(mine + (ii * 2 + cb) * 16 + 4 * q) =
                f32x4{acc[2 * r + ii][cb][4 * q], acc[2 * r + ii][cb][4 * q + 1], acc[2 * r + ii][cb][4 * q + 2],
                      acc[2 * r + ii][cb][4 * q + 3]};
        }
      __syncthreads();
      // All 12 reads first, then the sums in K-quarter order.
      f32x4 pk[4][4];
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          pk[k2][q] = k2 == KQC
                          ? f32x4{acc[2 * r + KQC / 2][KQC % 2][4 * q], acc[2 * r + KQC / 2][KQC % 2][4 * q + 1],
                                  acc[2 * r + KQC / 2][KQC % 2][4 * q + 2], acc[2 * r + KQC / 2][KQC % 2][4 * q + 3]}
                          : *reinterpret_cast<const f32x4*>(ep + ((4 * nh + k2) * 64 + lane) * DEPI + 16 * KQC + 4 * q);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 sum = ((pk[0][q] + pk[1][q]) + pk[2][q]) + pk[3][q];
        res[r][4 * q] = sum[0];
        res[r][4 * q + 1] = sum[1];
        res[r][4 * q + 2] = sum[2];
        res[r][4 * q + 3] = sum[3];
      }
      __syncthreads();
    }
  };
  switch (kq) {
    case 0: reduce(std::integral_constant<int, 0>{}); break;
    case 1: reduce(std::integral_constant<int, 1>{}); break;
    case 2: reduce(std::integral_constant<int, 2>{}); break;
    default: reduce(std::integral_constant<int, 3>{}); break;
  }

  // 6. Split K.  A workgroup parks its partial tile, waits until every
  //    store is complete (s_waitcnt, then the barrier) and only then counts
  //    its arrival (counters[t]), adding bit 8 + kh when it parked through
  //    its L2.  The last to arrive (count split - 1) thus finds every other
  //    part complete; it adds the parts in k-part order, so the result does
  //    not depend on arrival order, then clears the tile's words for the
  //    next launch.  Parking: when every part of the tile runs on this XCD,
  //    through its L2 (plain stores and loads); otherwise with the sc1 cache
  //    policy (written through to, and read from, the memory side, as
  //    agent-scope atomics are).  The arrival bits say which, so the reader
  //    always reads a part the way it was written.
  if (split > 1) {
    constexpr int SC1 = 16;  // cache-policy bit sc1
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(part + (size_t)t * split * DPART), 0, (int)(split * DPART * sizeof(float)), 0x00020000);
    // Part kh, wave, round r, quarter q, lane: 16 B.
    auto off = [&](int kk, int r, int q) {
      return (uint32_t)((((kk * 8 + wave) * 2 + r) * 4 + q) * 64 + lane) * 16u;
    };
    const bool local = dma_flags[1] != 0u;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = __builtin_bit_cast(u32x4, f32x4{res[r][4 * q], res[r][4 * q + 1], res[r][4 * q + 2], res[r][4 * q + 3]});
        if (local)
          __builtin_amdgcn_raw_buffer_store_b128(v, pr, off(kh, r, q), 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b128(v, pr, off(kh, r, q), 0, SC1);
      }
    __builtin_amdgcn_s_waitcnt(0);  // every store of this thread complete
    __syncthreads();
    if (tid == 0)
      dma_flags[0] = __hip_atomic_fetch_add(&counters[t], 1u + (local ? (256u << kh) : 0u), __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if ((dma_flags[0] & 255u) != (unsigned int)(split - 1)) return;
    const uint32_t l2_parts = dma_flags[0] >> 8;  // parked through this XCD's L2 (all parts run on it)
    // Part by part in k order; all 8 loads of a part are in flight at once.
    f32x4 sum[8];
    for (int kk = 0; kk < split; ++kk) {
      f32x4 pv[8];
      if (kk == kh) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pv[i] = f32x4{res[i >> 2][4 * (i & 3)], res[i >> 2][4 * (i & 3) + 1], res[i >> 2][4 * (i & 3) + 2],
                        res[i >> 2][4 * (i & 3) + 3]};
      } else if ((l2_parts >> kk) & 1u) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pv[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off(kk, i >> 2, i & 3), 0, 0));
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          pv[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off(kk, i >> 2, i & 3), 0, SC1));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sum[i] = kk == 0 ? pv[i] : sum[i] + pv[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) res[i >> 2][4 * (i & 3) + e] = sum[i][e];
    if (tid == 0) {
      __hip_atomic_store(&counters[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int kk = 0; kk < split; ++kk)
        __hip_atomic_store(&counters[kDmaXccOffset + t * split + kk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // 7. Store: res[r] is block (row block 2r + kq/2, column block kq%2) of N
  //    half nh: element e at row 32 rb + 8(e/4) + 4h + e%4, column l32.
  const int gcol = col0 + 64 * nh + 32 * (kq & 1) + l32;
  if (row0 + DBM <= m && col0 + DBN <= n) {
    // A whole tile inside Y: the lane's column and row half in the per-lane
    // offset, each element's row in the scalar one (no per-store address
    // arithmetic or checks).
    const __amdgpu_buffer_rsrc_t yr =
        __builtin_amdgcn_make_buffer_rsrc((void*)y, 0, (int)((uint32_t)m * (uint32_t)n * 2u), 0x00020000);
    const uint32_t lane_off = ((uint32_t)(row0 + 4 * h) * (uint32_t)n + (uint32_t)gcol) * 2u;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int rb = 2 * r + (kq >> 1);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t row_off = (uint32_t)(32 * rb + 8 * (e >> 2) + (e & 3)) * (uint32_t)n * 2u;
        __builtin_amdgcn_raw_buffer_store_b16(TT::from_f32(res[r][e]), yr, lane_off, row_off, 0);
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int rb = 2 * r + (kq >> 1);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int grow = row0 + 32 * rb + 8 * (e >> 2) + 4 * h + (e & 3);
      if (grow < m && gcol < n) y[(size_t)grow * n + gcol] = TT::from_f32(res[r][e]);
    }
  }
}

size_t dma_lds(int k, int gs, int split) {
  return std::max((size_t)DRING + (size_t)(k / split / gs) * (DBN * 4), (size_t)DEPI_BYTES);
}

}  // namespace

// K/split a multiple of 1024 and gs <= 128 make every group count and
// K-range start a multiple of 8 groups (the 16-B scale/bias loads).
bool qmm_dma_fits(int m, int n, int k, int gs, int bits, int split) {
  if (bits != 4 || split < 1 || k % (1024 * split) != 0 || gs > 128 || gs < 32) return false;
  if (k / split / gs > 8 * 4 * DMAXB) return false;
  if (dma_lds(k, gs, split) > (size_t)DLDS_MAX) return false;
  const uint64_t tiles = (uint64_t)((m + DBM - 1) / DBM) * ((n + DBN - 1) / DBN);
  if (split > 1 && (tiles > (uint64_t)kDmaMaxTiles || tiles * split > (uint64_t)kDmaMaxParts)) return false;
  const uint64_t xb = (uint64_t)m * k * 2, wb = (uint64_t)(n + DBN) * k / 2, yb = (uint64_t)m * n * 2;
  return xb < (1ull << 31) && wb < (1ull << 31) && yb < (1ull << 31);
}

int qmm_dma_split(int m, int n, int k, int gs, int bits, int cu_count) {
  const long tiles = (long)((m + DBM - 1) / DBM) * ((n + DBN - 1) / DBN);
  const long cus = cu_count > 0 ? cu_count : 256;
  int best = 0;
  long best_cost = 0;
  for (int split : {1, 2, 4}) {
    if (!qmm_dma_fits(m, n, k, gs, bits, split)) continue;
    // Makespan in k-units: rounds of one workgroup per CU, each K/split
    // deep plus a workgroup's fixed phases (prologue, K-quarter reduction,
    // store: about 2000 k-units of loop time), plus the partial-tile
    // exchange (about 4 stages) when split.  Fitted to measured splits:
    // config 3a (M = 512, N = 4096) 1 / 2 / 4 parts 30.3 / 27.1 / 38.7 us,
    // N = 12288 75.8 / 82.9 / 80.3 us, M = 2048 all within 2 %.
    const long rounds = (tiles * split + cus - 1) / cus;
    const long cost = rounds * (k / split + 2000) + (split > 1 ? 512 : 0);
    if (best == 0 || cost < best_cost) {
      best = split;
      best_cost = cost;
    }
  }
  return best;
}

size_t qmm_dma_scratch_bytes(int m, int n, int split) {
  if (split <= 1) return 0;
  const size_t tiles = (size_t)((m + DBM - 1) / DBM) * ((n + DBN - 1) / DBN);
  return kWideCounterBytes + tiles * split * DPART * sizeof(float);
}

hipError_t launch_qmm_dma(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                          void* scratch) {
  const int tiles_m = (m + DBM - 1) / DBM, tiles_n = (n + DBN - 1) / DBN;
  const size_t lds = dma_lds(k, q.gs, split);
  const int gs_shift = q.gs == 32 ? 5 : q.gs == 64 ? 6 : 7;
  unsigned int* counters = static_cast<unsigned int*>(scratch);
  float* part = scratch ? reinterpret_cast<float*>(static_cast<char*>(scratch) + kWideCounterBytes) : nullptr;
  if (split > 1 && !scratch) return hipErrorInvalidValue;
  auto run = [&](auto tag) -> hipError_t {
    using TT = decltype(tag);
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&qmm_dma_kernel<TT>);
      hipFuncAttributes fa;
      hipError_t e = hipFuncGetAttributes(&fa, fn);
      if (e != hipSuccess) return e;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((qmm_dma_kernel<TT>), dim3((unsigned)(tiles_m * tiles_n * split)), dim3(512), lds, s, q.w,
                       static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), m, n, k, gs_shift, tiles_m,
                       tiles_n, split, part, counters);
    return hipGetLastError();
  };
  if (q.dtype == CPQ_DTYPE_BF16) return run(BF16{});
  if (q.dtype == CPQ_DTYPE_F16) return run(F16{});
  return hipErrorInvalidValue;
}

}  // namespace cpq
