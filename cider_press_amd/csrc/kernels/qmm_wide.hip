// Prefill quantized GEMM, wide-tile kernel for gfx950 (4-bit weights).
//
// Reference op: affine_qmm_t / qmm_t_impl (kernels-mlx/mlx/backend/metal/
// kernels/quantized.h:1087-1213, 1713-1784), dispatched by
// crates/cider-press-kernels/src/kernels/qmm.rs:66-220.  Same numerics as
// every other path of this library: each weight is dequantized to T
// (RNE of fmaf(s, q, b)), products are accumulated in fp32 on the matrix
// cores, and the output is rounded to T once.
//
// Why a wide tile.  Per k, an output tile of BM x BN reads BM activations
// (2 B each) and BN weights (0.5 B each) into its CU.  A 128 x 64 tile moves
// about 70 B per CU-clock at the bf16 MFMA rate, more than the CU's
// global-to-LDS path sustains; 128 x 128 moves about half.  With few tiles
// (M = 512, N = 4096 gives 128), K is split over 2 or 4 workgroups so every
// CU has one; the partial tiles are summed by the workgroup that finishes
// last (below), in a fixed order.
//
// Matrix instruction: v_mfma_f32_32x32x16_{bf16,f16}.  Measured on MI355X,
// independent 32x32x16 MFMAs sustain about 2.1 PFLOP/s (bf16) against
// about 1.4 for 16x16x32, so the tile is built from 32 x 32 blocks.
// Layout: A[m][k] lane m%32 + 32(k/8), element k%8; B[k][n] lane
// n%32 + 32(k/8), element k%8; D[m][n] lane n + 32((m/4)%2), element
// 4(m/8) + m%4.
//
// Workgroup: 256 threads (4 waves, one per SIMD), tile 128 (M) x 128 (N),
// K range [kb0, kb0 + K/split) in stages of 128.
//   X: a ring of 4 LDS slots, each the 128 x 128 activation stage (32 KiB),
//      filled by buffer_load_dwordx4 ... lds four stages ahead; each copy
//      instruction moves 4 rows x 256 contiguous bytes; 16-B chunks are
//      XOR-swizzled by row so the MFMA-layout ds_read_b128 is conflict-free.
//      Slot indices are compile-time constants of the 8-stage unrolled loop.
//   Wave w owns the whole 128 x 128 tile for k-slice [32w, 32w + 32) of every
//   stage (two 16-k steps): 8 A fragments, 8 B operands, 32 MFMAs per stage,
//   256 fp32 accumulators per lane.  Each staged activation byte is read
//   from LDS once and each weight is dequantized once per workgroup.
//   W: per column block (32 columns) two 16-byte loads per lane every 4
//      stages: lane (c, h) loads the 32-element chunks of column 32jb + c
//      that wave w needs at stages 4G + 2h and 4G + 2h + 1; one
//      v_permlane32_swap per word pair then gives every lane half the 8
//      elements of each 16-k step of each stage (the natural operand layout,
//      so activations need no permutation).  Loads are spread over the
//      stages (one column block per stage) and land 1 to 4 stages before
//      their first use, in a two-group register ring.
//   Constants: the (s, b) pairs of the tile's columns and groups are staged
//      in LDS once as f32 b plus raw 16-bit s; the workgroup votes on the
//      fast dequantization (common.hpp), which then reads (s, b - 1024 s).
//   Schedule: each stage is software-pipelined in 32 slots (one MFMA each);
//      the dequantization of every B operand is cut into chunks issued
//      between the MFMAs two blocks after the operand's last read (so the
//      VALU work fills the matrix pipe's issue gaps).
//   Epilogue: the four K-slice partial tiles are summed through LDS in four
//      column passes, in wave order.  With split > 1 each workgroup stores
//      its partial tile, waits for the stores, and increments the tile's
//      arrival counter; the last to arrive adds the partials in k-part order
//      (so the result does not depend on arrival order), rounds, stores Y
//      and resets the counter to zero for the next launch.  No workgroup
//      waits on another.
#include <algorithm>

#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int WBM = 128, WBN = 128, WBK = 128;
constexpr int WNS = 4;                      // LDS ring slots (copies 4 stages ahead)
constexpr int WSLOT = WBM * WBK * 2;        // 32 KiB
constexpr int WEPI = 64 + 4;                // epilogue floats per lane (padded)
constexpr int WMAXB = 4;                    // 8-group constant blocks per thread: K/split/gs <= 64
constexpr int WLDS_MAX = 160 * 1024 - 512;  // dynamic LDS budget (static LDS of the vote aside)
constexpr int WPART = WBM * WBN;            // floats per partial tile
constexpr int WCST = 32 * 16 + 32 * 8;      // constants bytes per group: 32 lane columns x (4 f32 + 4 x 16-bit)

struct WideGeom {
  __amdgpu_buffer_rsrc_t xr, wr;
  uint32_t xoff[8];   // copy source offset of this lane for copy block j (stage 0 of the K range)
  uint32_t woff[4];   // weight offset of this lane for column block jb (group 0, first chunk)
  uint32_t a_off[2];  // A fragment offset of this lane for 16-k step t (row block 0) within a slot
  uint32_t cb_off;    // f32 b / c0 of this lane's columns (group 0)
  uint32_t cs_off;    // raw scales of this lane's columns (group 0)
  unsigned char* smem;
  int wave, gs_shift;
};

// Copy instruction J of stage s (rows 4(8*wave + J) .. +3) into ring slot `slot_index`.
template <int J>
__device__ __forceinline__ void wide_dma1(const WideGeom& g, int s, int slot_index) {
  unsigned char* slot = g.smem + (size_t)slot_index * WSLOT;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      g.xr, (__attribute__((address_space(3))) void*)(slot + (g.wave * 8 + J) * 1024), 16, g.xoff[J],
      s * (WBK * 2), 0, 0);
}

template <int J = 0>
__device__ __forceinline__ void wide_dma(const WideGeom& g, int s, int slot_index) {
  if constexpr (J < 8) {
    wide_dma1<J>(g, s, slot_index);
    wide_dma<J + 1>(g, s, slot_index);
  }
}

// Raw weights of group `grp` for column block JB: on lane half h the chunks
// of stages 4grp + 2h (entry 0) and 4grp + 2h + 1 (entry 1).
template <int JB>
__device__ __forceinline__ void wide_wload(const WideGeom& g, int grp, u32x4 (&wr)[4][2]) {
  wr[JB][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.woff[JB], grp * 256, 0));
  wr[JB][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(g.wr, g.woff[JB] + 64u, grp * 256, 0));
}

// Exchange between the lane halves: entry q (chunk of stage 4G + 2h + q on
// half h) becomes {k-step 0 word of stage q, of stage 2+q, k-step 1 word of
// stage q, of stage 2+q}, each word holding the 8 elements lane half h
// needs (elements 16t + 8h .. +7 of the stage's 32-element slice).
__device__ __forceinline__ void wide_xchg(u32x4& v) {
  const auto t01 = __builtin_amdgcn_permlane32_swap(v.x, v.y, false, false);
  const auto t23 = __builtin_amdgcn_permlane32_swap(v.z, v.w, false, false);
  v = u32x4{t01[0], t01[1], t23[0], t23[1]};
}

// acc += A . B on the matrix cores, with the accumulator pinned to AGPRs
// (dst == srcC).  Written as inline asm because the compiler does not keep
// 256 live accumulators in place across the loop (it rotates them through
// VGPRs and spills).  The compiler therefore cannot apply the MFMA hazard
// rules to these instructions; they are kept here instead:
//   - a VALU write of a VGPR (a dequantized B operand, or a register copy
//     the allocator places anywhere, e.g. at the loop back-edge) must be 2
//     wait states ahead of an MFMA read: the s_nop 1 in front of every MFMA
//     provides them, in the issue gap of the matrix pipe;
//   - A operands come from ds_read (the compiler waits on lgkmcnt);
//   - VALU / LDS readers of the results wait for the pipeline with
//     wide_mfma_drain.
template <typename TT>
__device__ __forceinline__ void wide_mfma(f32x16& acc, const u32x4& a, const u32x4& b) {
  if constexpr (Sig16<TT>::bf16)
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Wait states between the last MFMA writing an accumulator and the first
// VALU / LDS read of it (more than the 32x32x16 XDL result latency); each
// group of 8 accumulators passes through the wait before it is read.
__device__ __forceinline__ void wide_mfma_drain(f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; i += 2)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(acc[i][0]), "+a"(acc[i][1]), "+a"(acc[i][2]), "+a"(acc[i][3]), "+a"(acc[i + 1][0]),
                   "+a"(acc[i + 1][1]), "+a"(acc[i + 1][2]), "+a"(acc[i + 1][3]));
}

// 8 nibbles e0..e7 of one word (k order) -> MFMA B operand in k order.
// Fast path: v_and_or drops e_even into the mantissa of f16 1024 (0x6400,
// giving 1024 + e) and e_odd, left in place as 16e, into f16 64 (0x5400,
// giving 64 + e); one v_fma_mix_f32 each computes s*(1024 + e) + c0 with
// c0 = b - 1024 s, or s*(64 + e) + c1 with c1 = b - 64 s = c0 + 960 s:
// fmaf(s, e, b) exactly whenever c0 and c1 are exact (the workgroup vote).
// The constants arrive as f32 (s, c0); the slow path gets (s, b).
template <typename TT, bool FAST>
__device__ __forceinline__ u32x4 wide_dequant(uint32_t word, float sf, float cb) {
  if constexpr (FAST) {
    const float c1 = fmaf(960.f, sf, cb);
    const uint32_t w8 = word >> 8;
    const uint32_t p0 = and_or(word, 0x000F000Fu, 0x64006400u);  // (1024 + e0, 1024 + e4)
    const uint32_t p1 = and_or(word, 0x00F000F0u, 0x54005400u);  // (64 + e1, 64 + e5)
    const uint32_t p2 = and_or(w8, 0x000F000Fu, 0x64006400u);    // (1024 + e2, 1024 + e6)
    const uint32_t p3 = and_or(w8, 0x00F000F0u, 0x54005400u);    // (64 + e3, 64 + e7)
    return u32x4{TT::pack2(fmaf(sf, f16lo(p0), cb), fmaf(sf, f16lo(p1), c1)),
                 TT::pack2(fmaf(sf, f16lo(p2), cb), fmaf(sf, f16lo(p3), c1)),
                 TT::pack2(fmaf(sf, f16hi(p0), cb), fmaf(sf, f16hi(p1), c1)),
                 TT::pack2(fmaf(sf, f16hi(p2), cb), fmaf(sf, f16hi(p3), c1))};
  } else {
    const uint32_t wd[1] = {word};
    return dequant_slice_nat<TT, 4, false, 0>(wd, sf, sf * 0.0625f, cb, 0.f, 0.f);
  }
}

// The fast dequantization cut into 4 chunks, one per MFMA slot of a block, so
// the VALU work fills the matrix pipe's issue gaps.  The nibble extractions
// all go first: v_fma_mix reads its 16-bit source 2 wait states after the
// VALU write at the earliest, and with the MFMA slot in between no chunk
// needs a wait-state nop.
struct WideDeq {
  uint32_t word, w8, p0, p1, p2, p3, o0, o1, o2, o3;
  float sf, cb, c1, f0, f1, f2, f3, f4, f5, f6, f7;
};

template <typename TT, int K>
__device__ __forceinline__ void wide_deq_step(WideDeq& d) {
  if constexpr (K == 0) {
    d.c1 = fmaf(960.f, d.sf, d.cb);
    d.w8 = d.word >> 8;
    d.p0 = and_or(d.word, 0x000F000Fu, 0x64006400u);
    d.p1 = and_or(d.word, 0x00F000F0u, 0x54005400u);
    d.p2 = and_or(d.w8, 0x000F000Fu, 0x64006400u);
    d.p3 = and_or(d.w8, 0x00F000F0u, 0x54005400u);
  } else if constexpr (K == 1) {
    d.f0 = fmaf(d.sf, f16lo(d.p0), d.cb);
    d.f1 = fmaf(d.sf, f16lo(d.p1), d.c1);
    d.f4 = fmaf(d.sf, f16hi(d.p0), d.cb);
    d.f5 = fmaf(d.sf, f16hi(d.p1), d.c1);
  } else if constexpr (K == 2) {
    d.o0 = TT::pack2(d.f0, d.f1);
    d.o2 = TT::pack2(d.f4, d.f5);
    d.f2 = fmaf(d.sf, f16lo(d.p2), d.cb);
    d.f3 = fmaf(d.sf, f16lo(d.p3), d.c1);
  } else if constexpr (K == 3) {
    d.o1 = TT::pack2(d.f2, d.f3);
    d.f6 = fmaf(d.sf, f16hi(d.p2), d.cb);
    d.f7 = fmaf(d.sf, f16hi(d.p3), d.c1);
    d.o3 = TT::pack2(d.f6, d.f7);
  }
}

// Scale of column block jb from the 4 raw 16-bit scales of a lane.
template <typename TT>
__device__ __forceinline__ float wide_scale(const u32x2& sn, int jb) {
  const uint32_t w = sn[jb >> 1];
  return TT::to_f32((uint16_t)((jb & 1) ? (w >> 16) : (w & 0xffffu)));
}

// Source word of B operand o = 2*jb + t of a stage whose position in its
// weight group is T (ring entry already exchanged).
template <int T>
__device__ __forceinline__ uint32_t wide_word(const u32x4 (&wrg)[4][2], int o) {
  return wrg[o >> 1][T & 1][2 * (o & 1) + (T >> 1)];
}

// Issue pattern of stage P of an 8-stage block (the block base s0 is a
// multiple of 8), in this order (pinned by scheduling barriers):
//   copies for stage s+4, into the slot of stage s (whose fragments were
//   read during stage s-1), unless past the end;
//   weights: column block r = (P+1) & 3 of group ((s-3)>>2) + 2 (two
//   loads) into ring entry ((s-3)>>2) & 1, i.e. every stage one block of
//   the group after next, each loaded after the last dequantization that
//   read its ring entry and 1 to 4 stages before its first new use; none
//   past the last group (in the last block only P = 0..2 load).
// The prologue issues the same pattern for stages -5..-1: group 0, copies
// 0..3 and block 0 of group 1.
constexpr bool wide_wld_at(int p, bool tail) { return !tail || p < 3; }
constexpr bool wide_dma_at(int p, bool tail) { return !tail || p + 4 < 8; }
constexpr int wide_w(int p, bool tail) { return (p < 0 ? true : wide_wld_at(p, tail)) ? 2 : 0; }
constexpr int wide_d(int p, bool tail) { return (p < 0 ? true : wide_dma_at(p, tail)) ? 8 : 0; }

// Loads issued after stage s+1's copies (issued at stage P-3) up to the
// wait at stage P: weights at P-3, copies and weights at P-2 and P-1 (a
// negative index is the previous, full block or the prologue).
template <bool TAIL, int P>
constexpr int wide_vmcnt() {
  return wide_w(P - 3, TAIL) + wide_d(P - 2, TAIL) + wide_w(P - 2, TAIL) + wide_d(P - 1, TAIL) +
         wide_w(P - 1, TAIL);
}

// Wait for all but N vector-memory loads and for every LDS access of this wave.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// Constants of column block 3 (B operands 6, 7) of the current stage, read
// one stage earlier.
struct WideCur {
  float c3;
  uint32_t s3;
};

// Stage s = s0 + P.  On entry `a` holds stage s's A fragments, bop[0..5]
// stage s's B operands 0..5 (column blocks 0..2), and `cur` the constants
// of column block 3.  The stage proves stage s+1's copies complete (own
// vmcnt, then the barrier for the other waves') and its own fragment reads
// of stage s done (lgkmcnt), then runs 8 MFMA blocks (operand o = 2jb + t:
// column block jb, 16-k step t; 4 row blocks each).  Block o also issues,
// chunk by chunk between its MFMAs, one dequantization: operands 6, 7 of
// stage s in blocks 0, 1 and operand o-2 of stage s+1 in block o >= 2, so
// every B register is rewritten 8 MFMAs after its last read and read 8 or
// more MFMAs after its write; its last slot issues copy instruction o of
// stage s+4.  Blocks 6, 7 reload the A fragments of step 0, 1 for stage s+1
// after their last use; block 7 issues the two weight loads last (after
// every copy of the stage, which the vmcnt accounting relies on).
template <typename TT, bool TAIL, int P, int O = 0>
__device__ __forceinline__ void wide_fast_blocks(const WideGeom& g, int s, u32x4 (&wr)[2][4][2], u32x4 (&a)[4][2],
                                                 u32x4 (&bop)[8], f32x16 (&acc)[4][4], const WideCur& cur,
                                                 const f32x4& cn, const u32x2& sn, const unsigned char* slot) {
  if constexpr (O < 8) {
    constexpr bool NEXT = !TAIL || P + 1 < 8;
    constexpr bool DMA = wide_dma_at(P, TAIL);
    constexpr bool WLD = wide_wld_at(P, TAIL);
    constexpr int NB0 = (P >> 2) & 1, T0 = P & 3;
    constexpr int NB = ((P + 1) >> 2) & 1, T = (P + 1) & 3;
    constexpr int WR = (P + 1) & 3;
    constexpr int WB = ((P + 5) >> 2) & 1;
    constexpr int JB = O >> 1, TS = O & 1;
    constexpr bool HAS = O < 2 || NEXT;
    constexpr int TGT = O < 2 ? 6 + O : O - 2;  // target B register
    WideDeq d;
    if constexpr (HAS) {
      if constexpr (O < 2) {
        if constexpr (T0 == 0 && O == 0) {
          wide_xchg(wr[NB0][3][0]);
          wide_xchg(wr[NB0][3][1]);
        }
        d.word = wide_word<T0>(wr[NB0], TGT);
        d.sf = TT::to_f32((uint16_t)cur.s3);
        d.cb = cur.c3;
      } else {
        if constexpr (T == 0 && (TGT & 1) == 0) {
          wide_xchg(wr[NB][TGT >> 1][0]);
          wide_xchg(wr[NB][TGT >> 1][1]);
        }
        d.word = wide_word<T>(wr[NB], TGT);
        d.sf = wide_scale<TT>(sn, TGT >> 1);
        d.cb = cn[TGT >> 1];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wide_mfma<TT>(acc[i][JB], a[i][TS], bop[O]);
      if constexpr (HAS) {
        if (i == 0) wide_deq_step<TT, 0>(d);
        if (i == 1) wide_deq_step<TT, 1>(d);
        if (i == 2) wide_deq_step<TT, 2>(d);
        if (i == 3) {
          wide_deq_step<TT, 3>(d);
          bop[TGT] = u32x4{d.o0, d.o1, d.o2, d.o3};
        }
      }
      if constexpr (O >= 6 && NEXT) a[i][O - 6] = *reinterpret_cast<const u32x4*>(slot + g.a_off[O - 6] + i * 8192);
      if (i == 3) {
        if constexpr (DMA) wide_dma1<O>(g, s + 4, P & 3);
        if constexpr (O == 7 && WLD) {
          __builtin_amdgcn_sched_barrier(0);
          wide_wload<WR>(g, ((s - 3) >> 2) + 2, wr[WB]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wide_fast_blocks<TT, TAIL, P, O + 1>(g, s, wr, a, bop, acc, cur, cn, sn, slot);
  }
}

// Slow-path (generic dequantization) stage: same issue pattern and operand
// schedule, without the chunking.
template <typename TT, bool TAIL, int P, int O = 0>
__device__ __forceinline__ void wide_slow_blocks(const WideGeom& g, int s, u32x4 (&wr)[2][4][2], u32x4 (&a)[4][2],
                                                 u32x4 (&bop)[8], f32x16 (&acc)[4][4], const WideCur& cur,
                                                 const f32x4& cn, const u32x2& sn, const unsigned char* slot) {
  if constexpr (O < 8) {
    constexpr bool NEXT = !TAIL || P + 1 < 8;
    constexpr bool DMA = wide_dma_at(P, TAIL);
    constexpr bool WLD = wide_wld_at(P, TAIL);
    constexpr int NB0 = (P >> 2) & 1, T0 = P & 3;
    constexpr int NB = ((P + 1) >> 2) & 1, T = (P + 1) & 3;
    constexpr int WR = (P + 1) & 3;
    constexpr int WB = ((P + 5) >> 2) & 1;
    constexpr int JB = O >> 1, TS = O & 1;
    constexpr int TGT = O < 2 ? 6 + O : O - 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wide_mfma<TT>(acc[i][JB], a[i][TS], bop[O]);
      if constexpr (O >= 6 && NEXT) a[i][O - 6] = *reinterpret_cast<const u32x4*>(slot + g.a_off[O - 6] + i * 8192);
    }
    if constexpr (O < 2) {
      if constexpr (T0 == 0 && O == 0) {
        wide_xchg(wr[NB0][3][0]);
        wide_xchg(wr[NB0][3][1]);
      }
      bop[TGT] = wide_dequant<TT, false>(wide_word<T0>(wr[NB0], TGT), TT::to_f32((uint16_t)cur.s3), cur.c3);
    } else if constexpr (NEXT) {
      if constexpr (T == 0 && (TGT & 1) == 0) {
        wide_xchg(wr[NB][TGT >> 1][0]);
        wide_xchg(wr[NB][TGT >> 1][1]);
      }
      bop[TGT] = wide_dequant<TT, false>(wide_word<T>(wr[NB], TGT), wide_scale<TT>(sn, TGT >> 1), cn[TGT >> 1]);
    }
    if constexpr (DMA) wide_dma1<O>(g, s + 4, P & 3);
    if constexpr (O == 7 && WLD) {
      __builtin_amdgcn_sched_barrier(0);
      wide_wload<WR>(g, ((s - 3) >> 2) + 2, wr[WB]);
    }
    __builtin_amdgcn_sched_barrier(0);
    wide_slow_blocks<TT, TAIL, P, O + 1>(g, s, wr, a, bop, acc, cur, cn, sn, slot);
  }
}

template <typename TT, bool FAST, bool TAIL, int P>
__device__ __forceinline__ void wide_step(const WideGeom& g, int s, u32x4 (&wr)[2][4][2], u32x4 (&a)[4][2],
                                          u32x4 (&bop)[8], f32x16 (&acc)[4][4], WideCur& cur) {
  constexpr bool NEXT = !TAIL || P + 1 < 8;
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NEXT) {
    wait_vm_lgkm<wide_vmcnt<TAIL, P>()>();
    __builtin_amdgcn_s_barrier();
  }
  f32x4 cn = {0.f, 0.f, 0.f, 0.f};
  u32x2 sn = {0u, 0u};
  const unsigned char* slot = g.smem + (size_t)((P + 1) & 3) * WSLOT;
  if constexpr (NEXT) {
    const int grp = ((s + 1) * WBK + 32 * g.wave) >> g.gs_shift;
    cn = *reinterpret_cast<const f32x4*>(g.smem + g.cb_off + (size_t)grp * 512);
    sn = *reinterpret_cast<const u32x2*>(g.smem + g.cs_off + (size_t)grp * 256);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (FAST)
    wide_fast_blocks<TT, TAIL, P>(g, s, wr, a, bop, acc, cur, cn, sn, slot);
  else
    wide_slow_blocks<TT, TAIL, P>(g, s, wr, a, bop, acc, cur, cn, sn, slot);
  if constexpr (NEXT) cur = WideCur{cn[3], sn[1] >> 16};
}

template <typename TT, bool FAST, bool TAIL, int P = 0>
__device__ __forceinline__ void wide_eight(const WideGeom& g, int s0, u32x4 (&wr)[2][4][2], u32x4 (&a)[4][2],
                                           u32x4 (&bop)[8], f32x16 (&acc)[4][4], WideCur& cur) {
  if constexpr (P < 8) {
    wide_step<TT, FAST, TAIL, P>(g, s0 + P, wr, a, bop, acc, cur);
    wide_eight<TT, FAST, TAIL, P + 1>(g, s0, wr, a, bop, acc, cur);
  }
}

template <typename TT, bool FAST>
__device__ __forceinline__ void wide_loop(const WideGeom& g, int S, u32x4 (&wr)[2][4][2], f32x16 (&acc)[4][4]) {
  // Stage 0's copies are complete and visible (prologue wait + barrier).
  u32x4 a[4][2], bop[8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) a[i][t] = *reinterpret_cast<const u32x4*>(g.smem + g.a_off[t] + i * 8192);
  const int grp = (32 * g.wave) >> g.gs_shift;
  const f32x4 cn = *reinterpret_cast<const f32x4*>(g.smem + g.cb_off + (size_t)grp * 512);
  const u32x2 sn = *reinterpret_cast<const u32x2*>(g.smem + g.cs_off + (size_t)grp * 256);
#pragma unroll
  for (int jb = 0; jb < 3; ++jb) {
    wide_xchg(wr[0][jb][0]);
    wide_xchg(wr[0][jb][1]);
  }
#pragma unroll
  for (int o = 0; o < 6; ++o)
    bop[o] = wide_dequant<TT, FAST>(wide_word<0>(wr[0], o), wide_scale<TT>(sn, o >> 1), cn[o >> 1]);
  WideCur cur{cn[3], sn[1] >> 16};
  int s0 = 0;
  for (; s0 < S - 8; s0 += 8) wide_eight<TT, FAST, false>(g, s0, wr, a, bop, acc, cur);
  wide_eight<TT, FAST, true>(g, s0, wr, a, bop, acc, cur);
}

template <typename TT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void qmm_wide_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int m, int n, int k, int gs_shift, int tiles_m,
    int tiles_n, int split, float* __restrict__ part, unsigned int* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;

  // Workgroup order: each XCD (linear ids congruent mod 8) takes a
  // contiguous run of (tile, k-part) pairs, k-part fastest, then M tiles, so
  // the k-parts of a tile share one L2 and the run shares panels of X and W.
  const int nwg = tiles_m * tiles_n * split;
  int v = blockIdx.x;
  if ((nwg & 7) == 0) v = (v & 7) * (nwg >> 3) + (v >> 3);
  const int kh = v % split, t = v / split;
  const int mt = t % tiles_m, nt = t / tiles_m;
  const int row0 = mt * WBM, col0 = nt * WBN;
  const int KL = k / split, kb0 = kh * KL;
  const int S = KL / WBK;
  const int G = k >> gs_shift, GL = KL >> gs_shift, gk0 = kb0 >> gs_shift;
  const uint32_t rowbytes = (uint32_t)k / 2u;

  WideGeom g;
  g.smem = smem;
  g.wave = wave;
  g.gs_shift = gs_shift;
  g.xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)((uint32_t)m * (uint32_t)k * 2u), 0x00020000);
  g.wr = __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, (int)((uint32_t)n * rowbytes), 0x00020000);
  // Copy block b = 8*wave + j holds rows 4b .. 4b+3; lane i lands at row
  // 4b + i/16, physical chunk i%16, which holds logical chunk (i%16)^(row%16).
  // Rows past M re-read row M-1 (never stored).
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int rr = (wave * 8 + j) * 4 + (lane >> 4);
    const int c = (lane & 15) ^ (rr & 15);
    const int grow = min(row0 + rr, m - 1);
    g.xoff[j] = ((uint32_t)grow * (uint32_t)k + (uint32_t)kb0 + (uint32_t)(c * 8)) * 2u;
  }
  // A fragment of lane (l32, h), row block i, step t: row 32i + l32,
  // logical chunk 4*wave + 2t + h.
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) g.a_off[tt] = (uint32_t)(l32 * 256 + (((4 * wave + 2 * tt + h) ^ (l32 & 15)) * 16));
  // Weights of lane (l32, h), column block jb: column col0 + 32jb + l32,
  // chunk 16*grp + 8h + 4q + wave of the K range (q = 0, 1: +64 bytes).
  // Columns past N read zeros through the descriptor's range check (never
  // stored).
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
    g.woff[jb] = (uint32_t)(col0 + 32 * jb + l32) * rowbytes + (uint32_t)kb0 / 2u + (uint32_t)((8 * h + wave) * 16);
  const uint32_t cst_base = (uint32_t)WNS * WSLOT;
  g.cb_off = cst_base + (uint32_t)l32 * 16;
  g.cs_off = cst_base + (uint32_t)GL * 512 + (uint32_t)l32 * 8;

  // 1. Scale / bias words of the tile's columns: thread (column tid % 128,
  //    half tid / 128) loads 8-group blocks half, half + 2, ... (16-B loads;
  //    G, the K-range start and the pointers are 16-B aligned), issued first
  //    and consumed once the stream loads are in flight.
  const int cc = tid & 127, half = tid >> 7;
  const int ccol = min(col0 + cc, n - 1);
  u32x4 sv[WMAXB], bv[WMAXB];
#pragma unroll
  for (int u = 0; u < WMAXB; ++u) {
    const int gb = half + 2 * u;
    if (8 * gb < GL) {
      const size_t off = (size_t)ccol * G + gk0 + 8 * gb;
      sv[u] = *reinterpret_cast<const u32x4*>(scales + off);
      bv[u] = *reinterpret_cast<const u32x4*>(biases + off);
    }
  }

  // 2. Stream loads in the steady-state pattern of stages -5..-1.
  u32x4 wr[2][4][2];
  __builtin_amdgcn_sched_barrier(0);
  wide_wload<0>(g, 0, wr[0]);
  __builtin_amdgcn_sched_barrier(0);
  wide_dma(g, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  wide_wload<1>(g, 0, wr[0]);
  __builtin_amdgcn_sched_barrier(0);
  wide_dma(g, 1, 1);
  __builtin_amdgcn_sched_barrier(0);
  wide_wload<2>(g, 0, wr[0]);
  __builtin_amdgcn_sched_barrier(0);
  wide_dma(g, 2, 2);
  __builtin_amdgcn_sched_barrier(0);
  wide_wload<3>(g, 0, wr[0]);
  __builtin_amdgcn_sched_barrier(0);
  wide_dma(g, 3, 3);
  __builtin_amdgcn_sched_barrier(0);
  wide_wload<0>(g, 1, wr[1]);
  __builtin_amdgcn_sched_barrier(0);

  // 3. Constants into LDS: f32 c0 = b - 1024 s (fast dequantization) or b
  //    (generic) at [(group * 32 + c % 32) * 4 + c / 32] and the raw 16-bit
  //    scale at the same index of the scale array, for column col0 + c.
  //    Each thread checks its groups (packed exponent check, the exact
  //    predicate only when that one is inconclusive) and stores c0 if they
  //    pass, b if not; the workgroup then votes, and if the vote fails the
  //    threads that stored c0 store b instead.  With one wave per SIMD every
  //    instruction here costs several cycles, so the common path is kept to
  //    a few per group.
  float* cstb = reinterpret_cast<float*>(smem + cst_base);
  uint16_t* csts = reinterpret_cast<uint16_t*>(smem + cst_base + (size_t)GL * 512);
  const int cidx = (cc & 31) * 4 + (cc >> 5);
  FastQuick fq;
  fast_quick_init(fq);
#pragma unroll
  for (int u = 0; u < WMAXB; ++u)
    if (8 * (half + 2 * u) < GL)
#pragma unroll
      for (int q = 0; q < 4; ++q) fast_quick_add<TT>(fq, sv[u][q], bv[u][q]);
  bool ok = fast_quick_ok<TT>(fq);
  if (!ok) {
    ok = true;
#pragma unroll
    for (int u = 0; u < WMAXB; ++u)
      if (8 * (half + 2 * u) < GL)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ok &= fast_ok_bits<TT>(sv[u][q] & 0xffffu, bv[u][q] & 0xffffu) &
                fast_ok_bits<TT>(sv[u][q] >> 16, bv[u][q] >> 16);
  }
  auto store_constants = [&](bool c0, bool scales_too) {
#pragma unroll
    for (int u = 0; u < WMAXB; ++u) {
      const int gb = half + 2 * u;
      if (8 * gb < GL) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t s16 = (e & 1) ? sv[u][e >> 1] >> 16 : sv[u][e >> 1] & 0xffffu;
          const uint32_t b16 = (e & 1) ? bv[u][e >> 1] >> 16 : bv[u][e >> 1] & 0xffffu;
          const float b = TT::to_f32((uint16_t)b16);
          cstb[(8 * gb + e) * 128 + cidx] = c0 ? fmaf(-1024.f, TT::to_f32((uint16_t)s16), b) : b;
          if (scales_too) csts[(8 * gb + e) * 128 + cidx] = (uint16_t)s16;
        }
      }
    }
  };
  if (ok)
    store_constants(true, true);
  else
    store_constants(false, true);
  // Vote through one LDS word per wave.  This wave's stage-0 copies have
  // landed (4 x 8 younger loads may still be in flight); the barrier makes
  // every wave's copies, constants and vote visible.  A bare s_barrier after
  // explicit waits: a fenced barrier would also wait for the copies of
  // stages 1..3.
  __shared__ uint32_t wide_vote[4];
  const bool wave_ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
  if (lane == 0) wide_vote[wave] = wave_ok ? 1u : 0u;
  asm volatile("" ::: "memory");
  wait_vm_lgkm<32>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  const bool fast = (wide_vote[0] & wide_vote[1] & wide_vote[2] & wide_vote[3]) != 0u;
  if (!fast) {
    if (ok) store_constants(false, false);
    asm volatile("" ::: "memory");
    wait_vm_lgkm<63>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  // 4. Stream K.
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][jb][e] = 0.f;
  if (fast)
    wide_loop<TT, true>(g, S, wr, acc);
  else
    wide_loop<TT, false>(g, S, wr, acc);
  wide_mfma_drain(acc);

  // 5. Sum the four K-slice partial tiles in four column passes: pass p
  //    parks column block p of every wave (acc[i][p], i = 0..3); thread
  //    (wave, lane) then adds row block i = wave over the waves in order.
  __syncthreads();
  float* ep = reinterpret_cast<float*>(smem);
  f32x4 res[16];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float* mine = ep + (wave * 64 + lane) * WEPI;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(mine + 16 * i + 4 * q) =
            f32x4{acc[i][p][4 * q], acc[i][p][4 * q + 1], acc[i][p][4 * q + 2], acc[i][p][4 * q + 3]};
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 sum = *reinterpret_cast<const f32x4*>(ep + lane * WEPI + 16 * wave + 4 * q);
#pragma unroll
      for (int w2 = 1; w2 < 4; ++w2)
        sum += *reinterpret_cast<const f32x4*>(ep + (w2 * 64 + lane) * WEPI + 16 * wave + 4 * q);
      res[p * 4 + q] = sum;
    }
    __syncthreads();
  }

  // 6. Split K: park the partial, count arrivals; the last adds all parts in
  //    k-part order.  The partial tiles are the only data shared between
  //    workgroups, so they are stored and loaded with the agent-coherence
  //    cache policy (sc1: written through to / read from the memory side,
  //    as agent-scope atomic stores and loads are) and ordered by waiting
  //    for the stores before the arrival count -- no L2 writeback.
  if (split > 1) {
    constexpr int SC1 = 16;  // cache-policy bit sc1
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(part + (size_t)t * split * WPART), 0, (int)(split * WPART * sizeof(float)), 0x00020000);
    const uint32_t mine = (uint32_t)(kh * WPART + tid * 4) * 4u;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, res[r]), pr, mine + r * 4096u, 0, SC1);
    __builtin_amdgcn_s_waitcnt(0);  // every store of this thread complete
    __syncthreads();
    unsigned int* flag = reinterpret_cast<unsigned int*>(smem);
    if (tid == 0) flag[0] = __hip_atomic_fetch_add(&counters[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (flag[0] != (unsigned int)(split - 1)) return;
    const uint32_t base = (uint32_t)(tid * 4) * 4u;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t o = base + r * 4096u;
      auto ld = [&](int kk) {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, o + (uint32_t)kk * WPART * 4u, 0, SC1));
      };
      f32x4 sum = kh == 0 ? res[r] : ld(0);
      sum += kh == 1 ? res[r] : ld(1);
      if (split > 2) {
        sum += kh == 2 ? res[r] : ld(2);
        sum += kh == 3 ? res[r] : ld(3);
      }
      res[r] = sum;
    }
    if (tid == 0) __hip_atomic_store(&counters[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // 7. Store: res[4p + q] holds elements 4q .. 4q+3 of row block i = wave,
  //    column block p: rows 32*wave + 8q + 4h + e, column 32p + l32.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int p = r >> 2, q = r & 3;
    const int gcol = col0 + 32 * p + l32;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int grow = row0 + 32 * wave + 8 * q + 4 * h + e;
      if (grow < m && gcol < n) y[(size_t)grow * n + gcol] = TT::from_f32(res[r][e]);
    }
  }
}

__global__ void zero_words_kernel(unsigned int* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

size_t wide_lds(int k, int gs, int split) { return (size_t)WNS * WSLOT + (size_t)(k / split / gs) * WCST; }

}  // namespace

// K/split a multiple of 1024 and gs <= 128 make every group count and
// K-range start a multiple of 8 groups (the 16-B scale/bias loads).
bool qmm_wide_fits(int m, int n, int k, int gs, int bits, int split) {
  if (bits != 4 || split < 1 || k % (1024 * split) != 0 || gs > 128) return false;
  if (k / split / gs > 8 * 2 * WMAXB) return false;
  if (wide_lds(k, gs, split) > (size_t)WLDS_MAX) return false;
  // One arrival counter per tile at the head of the scratch.
  const uint64_t tiles = (uint64_t)((m + WBM - 1) / WBM) * ((n + WBN - 1) / WBN);
  if (split > 1 && tiles > kWideCounterBytes / 4) return false;
  const uint64_t xb = (uint64_t)m * k * 2, wb = (uint64_t)(n + WBN) * k / 2;
  return xb < (1ull << 31) && wb < (1ull << 31);
}

size_t qmm_wide_scratch_bytes(int m, int n, int split) {
  if (split <= 1) return 0;
  const size_t tiles = (size_t)((m + WBM - 1) / WBM) * ((n + WBN - 1) / WBN);
  return kWideCounterBytes + tiles * split * WPART * sizeof(float);
}

int qmm_wide_split(int m, int n, int k, int gs, int bits, int cu_count) {
  const long tiles = (long)((m + WBM - 1) / WBM) * ((n + WBN - 1) / WBN);
  const long cus = cu_count > 0 ? cu_count : 256;
  int best = 0;
  long best_cost = 0;
  for (int split : {1, 2, 4}) {
    if (!qmm_wide_fits(m, n, k, gs, bits, split)) continue;
    // Makespan in k-units: rounds of one workgroup per CU, each K/split
    // deep, plus the partial-tile exchange (about 4 stages) when split.
    const long rounds = (tiles * split + cus - 1) / cus;
    const long cost = rounds * (k / split) + (split > 1 ? 512 : 0);
    if (best == 0 || cost < best_cost) {
      best = split;
      best_cost = cost;
    }
  }
  return best;
}

hipError_t launch_qmm_wide(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                           int split, void* scratch) {
  const int tiles_m = (m + WBM - 1) / WBM, tiles_n = (n + WBN - 1) / WBN;
  const size_t lds = std::max(wide_lds(k, q.gs, split), (size_t)4 * 64 * WEPI * 4);
  const int gs_shift = q.gs == 32 ? 5 : q.gs == 64 ? 6 : 7;
  unsigned int* counters = static_cast<unsigned int*>(scratch);
  float* part = scratch ? reinterpret_cast<float*>(static_cast<char*>(scratch) + kWideCounterBytes) : nullptr;
  if (split > 1 && !scratch) return hipErrorInvalidValue;
  auto run = [&](auto tag) -> hipError_t {
    using TT = decltype(tag);
    static const hipError_t attr = [] {
      const void* fn = reinterpret_cast<const void*>(&qmm_wide_kernel<TT>);
      hipFuncAttributes fa;
      hipError_t e = hipFuncGetAttributes(&fa, fn);
      if (e != hipSuccess) return e;
      return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(160 * 1024 - fa.sharedSizeBytes));
    }();
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((qmm_wide_kernel<TT>), dim3((unsigned)(tiles_m * tiles_n * split)), dim3(256), lds, s,
                       q.w, static_cast<const uint16_t*>(q.scales), static_cast<const uint16_t*>(q.biases),
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(y), m, n, k, gs_shift, tiles_m,
                       tiles_n, split, part, counters);
    return hipGetLastError();
  };
  if (q.dtype == CPQ_DTYPE_BF16) return run(BF16{});
  if (q.dtype == CPQ_DTYPE_F16) return run(F16{});
  return hipErrorInvalidValue;
}

hipError_t zero_words(hipStream_t s, void* p, size_t n_words) {
  hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, s, static_cast<unsigned int*>(p), n_words);
  return hipGetLastError();
}

}  // namespace cpq
