// Streaming main loop of the verify-path matmuls (fast path).
//
// A workgroup of WV (4 or 8) wavefronts owns a block of NB = 64 weight rows
// (four 16-row MFMA tiles) and a range of K steps of CK = 64*WV k.  Cost
// model (measured on MI355X):
//
//   * a CU's vector memory pipeline retires roughly one cache-line request
//     every few cycles however few bytes of the line an instruction uses, so
//     every global read is a whole-line request: weights (whole 32*WV-byte
//     row pieces), activations (whole rows) and scales / biases (each row's
//     window for the whole K range, contiguous across rows when the range is
//     all of K) go straight to LDS with buffer_load ... lds, the steps
//     DEPTH - 1 ahead and the scales / biases once before the first step;
//   * the loop is VALU-issue bound (a SIMD retires one wave64 VALU op per
//     ~4.2 cycles), so every address is computed once per lane: a DMA is an
//     SGPR base (advanced by scalar adds) plus a lane-constant VGPR offset,
//     and the fragment reads of a step cost one VGPR add per LDS region, the
//     rest being immediate offsets;
//   * LDS read latency is hidden by register double buffering: the fragments
//     of step c+1 are read from LDS while step c is computed, and WV = 8 puts
//     two wavefronts on every SIMD to overlap the remaining stalls;
//   * each wavefront takes a 64-k slice of every step for all four tiles, so
//     the activation stage is read from LDS once per workgroup (not once per
//     wavefront) and its group sums cost two MFMAs per slice;
//   * every LDS layout is XOR-swizzled per row so the fragment reads spread
//     over the banks.
//
// Arithmetic (per lane, tile t, M-block mt): P = sum over the slice of
// x * (OFF + q) by 16x16x32 MFMAs (weights from dequant_word4, activations
// unconverted), X = sum of x over the slice by an MFMA against ones (its
// output layout matches the accumulator's), then
//     acc += s * P + (b - OFF * s) * X
// per quantisation group.  A slice never straddles a group boundary at
// gs = 64 or 128 (gs = 128: a slice is half a group, and both terms are
// linear in the slice), and covers exactly two groups at gs = 32.
//
// Synchronisation: LDS DMA loads are tracked by vmcnt only, and the compiler
// does not know that a later ds_read depends on them, so the loop waits with
// an explicit s_waitcnt vmcnt(n) (n = loads this wavefront issued after the
// step it needs) followed by a workgroup barrier, once per step.  The same
// barrier (with lgkmcnt(0)) proves that every wavefront has finished reading
// the stage the next DMA overwrites.
#pragma once

#include "dfmi_core.h"

namespace dfmi {

constexpr int kStreamRows = 64;   // weight rows per workgroup
constexpr int kStreamTiles = 4;   // 16-row MFMA tiles per workgroup, all in every wavefront
constexpr uint32_t kNoRow = 0x80000000u;  // buffer offset past the end of every buffer
// Scale / bias window of a run() call: at most SBPC 16-byte pieces (8
// groups each) per row and array, so a K range of at most sb_max_groups(SBPC)
// quantisation groups whatever its first group (a window may start
// mid-piece).
constexpr int kSbPieces = 16;
constexpr int sb_max_groups(int sbpc) { return 8 * (sbpc - 1); }

// Wait until at most N vector-memory operations of this wavefront are
// outstanding and all LDS operations are done, then the workgroup barrier.
// (gfx9 s_waitcnt encoding: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14,
// expcnt bits 6:4 left at max, lgkmcnt bits 11:8 = 0.)  A plain
// __syncthreads() would also wait for every outstanding load (vmcnt(0)),
// draining the DMA pipeline; the empty asm keeps the compiler from moving LDS
// accesses across the barrier.
template <int N>
__device__ inline void stage_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// stage_barrier<n> for a runtime n (clamped to 15: waiting longer is safe)
__device__ inline void stage_barrier_n(int n) {
  switch (n < 0 ? 0 : (n > 15 ? 15 : n)) {
    case 0: stage_barrier<0>(); break;
    case 1: stage_barrier<1>(); break;
    case 2: stage_barrier<2>(); break;
    case 3: stage_barrier<3>(); break;
    case 4: stage_barrier<4>(); break;
    case 5: stage_barrier<5>(); break;
    case 6: stage_barrier<6>(); break;
    case 7: stage_barrier<7>(); break;
    case 8: stage_barrier<8>(); break;
    case 9: stage_barrier<9>(); break;
    case 10: stage_barrier<10>(); break;
    case 11: stage_barrier<11>(); break;
    case 12: stage_barrier<12>(); break;
    case 13: stage_barrier<13>(); break;
    case 14: stage_barrier<14>(); break;
    default: stage_barrier<15>(); break;
  }
}


// Dynamic LDS of the streaming kernels (one allocation per workgroup).
extern __shared__ __attribute__((aligned(16))) char dfmi_smem[];

// 16 bytes per lane from a buffer (lane-constant VGPR offset + wave-uniform
// SGPR offset: no vector arithmetic per load) to LDS (wave-uniform
// destination; lane l lands at dst + 16 l).  CPOL: the load's cache-policy
// bits.
typedef __attribute__((address_space(3))) void lds_void;
template <int CPOL = 0>
__device__ inline void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lane_off, uint32_t uni_off,
                             char* lds_uniform) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)lds_uniform, 16, lane_off, uni_off, 0,
                                           CPOL);
}
// Non-temporal (gfx950 cache-policy bit NT) for the streams a launch reads
// once -- packed weights, pair tables, scale / bias windows -- so that they
// do not displace the lines that are read again (the activations every
// workgroup stages).  Measured on MI355X, graph replays A/B on one box: 27B
// sweep 3.652 -> 3.550 ms, 9B 1.393 -> 1.364 ms, fused lm_head 92.6 -> 87.4
// us, MoE 40 layers 2.189 -> 2.085 ms; the device-scope bit (SC1) alone
// changed nothing.
constexpr int kCpolStream = 2;

// A wave-uniform value the compiler may not split into constant parts (so a
// region base stays in one SGPR and the per-tile offsets fit the 16-bit
// ds_read immediate).
__device__ inline uint32_t opaque(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}

// RW row groups: the workgroup's WV wavefronts are RW groups of KW = WV / RW;
// group r owns rows 64 r .. 64 r + 63 of the block (NB = 64 RW rows), and
// wavefront k of a group takes the k-th 64-k slice of every step (CK = 64 KW
// k).  All groups read the same activation stage, so two groups halve the
// activation bytes per weight byte.
//
// TSB (pair streaming): instead of a scale / bias window loaded before the
// first step, every step's DMA brings the (scale, bias) pairs of its groups
// from a [K/GS][N] table of 32-bit pairs (scale in the low half, bias in the
// high half; dfmi_sb_pairs builds it): 64 GPC rows x 4 bytes per 64-row block
// and step, contiguous, so whole-line requests with no window in LDS (51 KB
// instead of 80 KB with 4 wavefronts: three workgroups per CU).  The
// arithmetic is the window path's, operation for operation.
template <typename Tag, int GS, int MT, int WV, int SBPC = kSbPieces, int BITS = 4, int RW = 1,
          bool TSB = false>
struct Stream {
  static constexpr int NT = kStreamTiles;   // 16-row tiles per wavefront
  static constexpr int KW = WV / RW;        // wavefronts along k
  static constexpr int NB = kStreamRows * RW;
  static constexpr int CK = 64 * KW;        // k per step
  static constexpr int GPC = CK / GS;       // quantisation groups per step
  static constexpr int XROW = CK * 2;       // bytes of one activation row per step
  static constexpr int XPPR = CK / 8;       // 16-byte pieces per activation row
  static constexpr int WPK = BITS / 4;      // 32-bit words per 8-k piece of a weight row
  static constexpr int WROW = CK * BITS / 8;  // bytes of one weight row per step
  static constexpr int WPPR = WROW / 16;    // 16-byte pieces per weight row
  // weight-stage swizzle key: row % SWZ (at most 16, so a tile's rows share
  // the keys of tile 0 whatever the row length)
  static constexpr int SWZ = WPPR < 16 ? WPPR : 16;
  static_assert(WV == 4 || WV == 8, "wavefronts");
  static_assert(BITS == 4 || BITS == 8, "weight bits");
  static_assert(RW == 1 || (RW == 2 && WV == 8 && MT == 1 && BITS == 4), "row groups");
  // 8-bit values are dequantised exactly: bf16 by conversion (no offset),
  // f16 by the 1024 magic
  static constexpr float OFFQ =
      BITS == 4 ? Num<Tag>::OFF : (std::is_same<Tag, BF16>::value ? 0.f : 1024.f);
  // LDS stages (DEPTH - 1 steps in flight).  Four stages with 8 wavefronts
  // measured slower than three on MI355X (4096x12288: 12.8 us vs 11.4 us):
  // the extra step in flight does not raise the per-CU request rate, and the
  // longer wait chain delays the first MFMA.  Two activation blocks (MT = 2)
  // with 4-bit weights take two stages: 80 KB, so two workgroups share a CU
  // and each one's wait is the other's compute (27B-class sweep at M = 32:
  // 7.59 ms vs 8.28 ms with three stages and one workgroup per CU).  8-bit
  // weights with one activation block and 4 wavefronts likewise fit 80 KB in
  // two stages; with two blocks they would still need 96 KB (one workgroup
  // per CU), so they keep three.
  // Two row groups take four stages with a scale window (160 KB, one
  // workgroup per CU) and three with pair streaming (78 KB, two per CU).
  static constexpr int DEPTH =
      RW == 2 ? (TSB ? 3 : 4)
              : ((MT == 2 && BITS == 4) || (MT == 1 && BITS == 8 && WV == 4) ? 2 : 3);
  // gs >= 64: a lane's two k-blocks take adjacent words (one 8-byte LDS read);
  // gs = 32: k-block j is group 2*wave + j, so the blocks stay group-pure.
  static constexpr bool PAIR = GS >= 64;
  static constexpr int XBUF = MT * 16 * XROW;  // bytes of one activation stage
  static constexpr int WBUF = NB * WROW;       // bytes of one weight stage
  // Scales and biases of the whole K range of a run() call, loaded once
  // before its first step: [array][row][SBP bytes], a row's window of 16-byte
  // pieces (8 groups each) XOR-swizzled by row.  Up to SBPC pieces, i.e. a
  // K range of at most MAX_GROUPS groups (any start).
  // (4 pieces only for windows that start at group 0: K / GS <= 32)
  static_assert(SBPC == 4 || SBPC == 8 || SBPC == 16, "scale window pieces");
  static constexpr int MAX_GROUPS = sb_max_groups(SBPC);
  static constexpr int SBPC_N = SBPC;         // pieces per row and array
  static constexpr int SBP = 16 * SBPC;        // bytes per row and array
  static constexpr int SBBUF = TSB ? 0 : 2 * NB * SBP;   // scales, then biases
  // TSB: one stage's pairs, [group of the step][row] 32-bit words; every
  // wavefront brings TPB bytes of them per step (one DMA, TLANES lanes)
  static_assert(!TSB || (PAIR && BITS == 4), "pair streaming: gs >= 64, 4-bit weights");
  static constexpr int SBS = TSB ? GPC * NB * 4 : 0;
  static constexpr int TPB = SBS / WV;
  static constexpr int TLANES = TPB / 16;
  // Scale / bias region first: its fragment reads use immediate offsets
  // (the ds_read offset field is 16 bits).
  static constexpr int SB_OFF = 0;
  static constexpr int X_OFF = SBBUF;
  static constexpr int W_OFF = X_OFF + DEPTH * XBUF;
  static constexpr int T_OFF = W_OFF + DEPTH * WBUF;
  static constexpr int LDS_BYTES = T_OFF + DEPTH * SBS;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
  // epilogue: [wave][t][mt][reg][lane] floats, aliasing the stages
  static constexpr int RED_FLOATS = NT * MT * 4 * 64;
  static_assert(WV * RED_FLOATS * 4 <= LDS_BYTES, "reduction buffer");
  // DMA instructions (1 KiB each) per wavefront
  static constexpr int X_DMA = XBUF / 1024 / WV;    // = 2 * MT
  static constexpr int W_DMA = WBUF / 1024 / WV;    // = 2
  static constexpr int SB_DMA = SBBUF / 1024 / WV;  // 2 SBPC / WV, once per run()
  static constexpr int SB_RPI = 1024 / SBP;         // rows per scale / bias instruction
  static constexpr int T_DMA = TSB ? 1 : 0;                 // pair DMA per step (TSB)
  static constexpr int CHUNK_DMA = X_DMA + W_DMA + T_DMA;
  static_assert(GS == 32 || GS == 64 || GS == 128, "group size");

  struct Ctx {
    __amdgpu_buffer_rsrc_t x, w, s, b;  // activations, packed weights, scales, biases
    __amdgpu_buffer_rsrc_t t;           // TSB: [K/GS][N] (scale, bias) pairs
    // Rows >= split of the block come from a second weight set (row - split):
    // the up projection next to the gate projection of a fused SwiGLU.
    __amdgpu_buffer_rsrc_t w2, s2, b2;
    const int32_t* xrows;  // activation row of local row m: xrows[m], or xbase + m if null
    int xbase;
    int split;   // NB: one weight set
    int K, M, N;
    int groups;  // K / GS
    int n0;      // first weight row of this workgroup (in each weight set)
    int wave, lane;
    uint32_t sb_base;  // LDS offset of this run's scale / bias window (past SB_OFF)
    // TSB: the pair table's row length in columns (0: N) and this matrix's
    // first column in it (several matrices' tables side by side)
    uint32_t tn, tc;

    // Dense defaults: activation rows 0 .. M-1, one weight set, its own
    // pair table.
    __device__ inline void dense() {
      xrows = nullptr;
      xbase = 0;
      split = NB;
      w2 = w;
      s2 = s;
      b2 = b;
      sb_base = 0;
      tn = 0;
      tc = 0;
    }
    __device__ inline uint32_t t_stride() const { return tn ? tn : (uint32_t)N; }
  };

  // Lane-constant offsets, computed once.
  struct Lane {
    uint32_t xg[X_DMA];  // activation DMA: byte offset in x of this lane's piece at step 0
    uint32_t wg[W_DMA];  // weight DMA: byte offset in w at step 0
    uint32_t xo[2];      // activation fragment j: byte offset inside a stage (M-block 0)
    uint32_t wo[2];      // weight fragment (j = 0; j = 1 too at gs = 32): offset inside a stage (tile 0)
    uint32_t sbr;        // scale fragment: row offset (tile 0)
    uint32_t swz;        // scale window swizzle key of this lane's row: col % SBPC
    uint32_t hsel;       // v_perm selector moving this wavefront's 16-bit half to the high half
    uint32_t tg;         // TSB: byte offset in the pair table of this lane's piece at step 0
    uint32_t tfo;        // TSB: pair fragment offset inside a stage (tile 0)
  };

  // One step's operands of this lane, read from LDS.
  struct Frag {
    u32x4 x[MT][2];           // activations of k-block j
    uint32_t w[NT][2 * WPK];  // packed words of k-block j: w[t][WPK j .. WPK j + WPK - 1]
    uint32_t sv[NT];    // dword holding this lane's scale(s)
    uint32_t bv[NT];    // dword holding this lane's bias(es)
  };

  // word (= 8-k piece) of the step that lane group kg of the wavefront with
  // k index kw feeds k-block j with
  __device__ static inline int piece_of(int kw, int kg, int j) {
    return PAIR ? 8 * kw + 2 * kg + j : 8 * kw + 4 * j + kg;
  }

  __device__ static inline Lane lane_setup(const Ctx& cx) {
    Lane L;
    const int col = cx.lane & 15, kg = cx.lane >> 4;
    // activation stage: instruction j covers 64 / XPPR consecutive rows; lane
    // l loads piece (l % XPPR) ^ (row & 15) of its row into slot l % XPPR.
    // Rows >= M take an offset past the end of the buffer: the range check
    // returns zeros without a memory request (their outputs are never
    // stored).  kNoRow + any step offset stays below 2^32, and every x
    // buffer the kernels take is smaller than 2^31 bytes.
#pragma unroll
    for (int i = 0; i < X_DMA; ++i) {
      const int j = cx.wave * X_DMA + i;
      const int r = j * (64 / XPPR) + cx.lane / XPPR;
      const int piece = (cx.lane % XPPR) ^ (r & 15);
      const int m = min(r, cx.M - 1);
      const int xr = cx.xrows ? cx.xrows[m] : cx.xbase + m;
      L.xg[i] = r < cx.M ? (uint32_t)xr * (uint32_t)cx.K * 2u + (uint32_t)piece * 16u : kNoRow;
    }
    // weight stage: instruction i of wavefront w covers 64 / WPPR consecutive
    // rows; lane l loads piece (l % WPPR) ^ (row % SWZ) of its row into slot
    // l % WPPR; rows >= N re-read row N-1
    constexpr int RPI = 64 / WPPR;
#pragma unroll
    for (int i = 0; i < W_DMA; ++i) {
      const int r = (cx.wave * W_DMA + i) * RPI + cx.lane / WPPR;
      const int piece = (cx.lane % WPPR) ^ (r % SWZ);
      const int n = min(cx.n0 + (r >= cx.split ? r - cx.split : r), cx.N - 1);
      L.wg[i] = (uint32_t)n * (uint32_t)(cx.K / 8 * BITS) + (uint32_t)piece * 16u;
    }
    // fragment reads (row m = col of M-block 0, row r = col of tile 0 of the
    // wavefront's row group; the other blocks / tiles are whole-row multiples
    // away; SWZ and SBPC divide 64, so the group's rows keep the keys of col)
    const int kw = cx.wave % KW, rg = cx.wave / KW;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      L.xo[j] = (uint32_t)(col * XROW + ((piece_of(kw, kg, j) ^ col) * 16));
      const int byte = piece_of(kw, kg, j) * 4 * WPK;
      L.wo[j] = (uint32_t)((64 * rg + col) * WROW + (((byte >> 4) ^ (col % SWZ)) * 16) +
                           (byte & 15));
    }
    L.sbr = (uint32_t)((64 * rg + col) * SBP);
    L.swz = (uint32_t)(col % SBPC);
    const int half = PAIR ? (((kw * 64) / GS) & 1) : 0;
    L.hsel = half ? 0x03020c0cu : 0x01000c0cu;
    if constexpr (TSB) {
      // lane l < TLANES of wavefront w brings stage bytes w TPB + 16 l: group
      // o / (4 NB) of the step, rows (o % (4 NB)) / 4 .. + 3 (rows past N read
      // past the table: zeros, never stored); lanes past TLANES are masked off
      const int o = cx.wave * TPB + 16 * cx.lane;
      const int grp = o / (4 * NB), row = (o % (4 * NB)) / 4;
      const int n = cx.n0 + row;
      L.tg = (cx.lane < TLANES && n < cx.N)
                 ? ((uint32_t)grp * cx.t_stride() + cx.tc + (uint32_t)n) * 4u
                 : kNoRow;
      L.tfo = (uint32_t)(((kw * 64 / GS) * NB + 64 * rg + col) * 4);
    } else {
      L.tg = 0;
      L.tfo = 0;
    }
    return L;
  }

  __device__ static inline void issue_x(const Ctx& cx, const Lane& L, int c, int stage) {
    const uint32_t u = (uint32_t)c * (uint32_t)(CK * 2);
#pragma unroll
    for (int i = 0; i < X_DMA; ++i)
      dma16(cx.x, L.xg[i], u, dfmi_smem + X_OFF + stage * XBUF + (cx.wave * X_DMA + i) * 1024);
  }

  __device__ static inline void issue_w(const Ctx& cx, const Lane& L, int c, int stage) {
    const uint32_t u = (uint32_t)c * (uint32_t)WROW;
    constexpr int RPI = 64 / WPPR;
#pragma unroll
    for (int i = 0; i < W_DMA; ++i) {
      const int r0 = (cx.wave * W_DMA + i) * RPI;  // wave-uniform
      dma16<kCpolStream>(r0 >= cx.split ? cx.w2 : cx.w, L.wg[i], u,
            dfmi_smem + W_OFF + stage * WBUF + r0 * WROW);
    }
  }

  // Scale / bias window: pieces [piece0, piece0 + P) (8 groups each) of
  // every row and array.  Instruction j of the workgroup covers array
  // j / (NB / SB_RPI), rows r0 .. r0 + SB_RPI - 1; lane l takes slot
  // l % SBPC of row r0 + l / SBPC, which holds piece
  // piece0 + (slot ^ (row % SBPC)).  Slots past the window, and rows past N,
  // read past the end of the buffer (zeros, no memory request).
  __device__ static inline void issue_sb(const Ctx& cx, int piece0, int P) {
#pragma unroll
    for (int i = 0; i < SB_DMA; ++i) {
      const int j = cx.wave * SB_DMA + i;  // wave-uniform
      const int arr = j / (NB / SB_RPI);
      const int r0 = (j % (NB / SB_RPI)) * SB_RPI;
      const int r = r0 + cx.lane / SBPC;
      const int q = (cx.lane % SBPC) ^ (r % SBPC);
      const bool second = r0 >= cx.split;  // wave-uniform (split is a multiple of SB_RPI)
      const int n = cx.n0 + (second ? r - cx.split : r);
      const uint32_t off =
          (q < P && n < cx.N)
              ? ((uint32_t)n * (uint32_t)cx.groups + (uint32_t)(piece0 + q) * 8u) * 2u
              : kNoRow;
      const __amdgpu_buffer_rsrc_t src = arr ? (second ? cx.b2 : cx.b) : (second ? cx.s2 : cx.s);
      dma16<kCpolStream>(src, off, 0u, dfmi_smem + SB_OFF + cx.sb_base + arr * NB * SBP + r0 * SBP);
    }
  }

  // TSB: step c's pairs (groups c GPC .. c GPC + GPC - 1 of the block's rows)
  __device__ static inline void issue_t(const Ctx& cx, const Lane& L, int c, int stage) {
    if (cx.lane < TLANES)
      dma16<kCpolStream>(cx.t, L.tg, (uint32_t)c * (uint32_t)(GPC * 4) * cx.t_stride(),
            dfmi_smem + T_OFF + stage * SBS + cx.wave * TPB);
  }

  __device__ static inline void issue_chunk(const Ctx& cx, const Lane& L, int c, int stage) {
    issue_x(cx, L, c, stage);
    issue_w(cx, L, c, stage);
    if constexpr (TSB) issue_t(cx, L, c, stage);
  }

  // Step c's fragments of this lane from LDS stage `stage`; g0w = first
  // group of the scale window (a multiple of 8).
  __device__ static inline void read_frag(const Ctx& cx, const Lane& L, int c, int stage, int g0w,
                                          Frag& f) {
    const uint32_t xb = opaque((uint32_t)(X_OFF + stage * XBUF));
    const uint32_t wb = opaque((uint32_t)(W_OFF + stage * WBUF));
    const char* xs0 = dfmi_smem + (L.xo[0] + xb);
    const char* xs1 = dfmi_smem + (L.xo[1] + xb);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f.x[mt][0] = *reinterpret_cast<const u32x4*>(xs0 + mt * 16 * XROW);
      f.x[mt][1] = *reinterpret_cast<const u32x4*>(xs1 + mt * 16 * XROW);
    }
    const char* ws0 = dfmi_smem + (L.wo[0] + wb);
    const char* ws1 = dfmi_smem + (L.wo[1] + wb);
    // this step's group in the window: piece gr / 8 (stored at slot
    // (gr / 8) ^ (col % SBPC)), dword (gr % 8) / 2 of the piece
    const int kw = cx.wave % KW;
    const uint32_t gr = (uint32_t)(c * GPC + (PAIR ? (kw * 64) / GS : 2 * kw) - g0w);
    const char* sbp = dfmi_smem + SB_OFF + cx.sb_base +
                      (L.sbr + (((gr >> 3) ^ L.swz) << 4) + ((gr & 7) >> 1) * 4);
    const char* tp = dfmi_smem + (L.tfo + opaque((uint32_t)(T_OFF + stage * SBS)));
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (PAIR && BITS == 4) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(ws0 + t * 16 * WROW);
        f.w[t][0] = v.x;
        f.w[t][1] = v.y;
      } else if constexpr (PAIR) {  // 8-bit: both k-blocks in one 16-byte piece
        const u32x4 v = *reinterpret_cast<const u32x4*>(ws0 + t * 16 * WROW);
        f.w[t][0] = v.x;
        f.w[t][1] = v.y;
        f.w[t][2] = v.z;
        f.w[t][3] = v.w;
      } else if constexpr (BITS == 4) {
        f.w[t][0] = *reinterpret_cast<const uint32_t*>(ws0 + t * 16 * WROW);
        f.w[t][1] = *reinterpret_cast<const uint32_t*>(ws1 + t * 16 * WROW);
      } else {
        const u32x2 v0 = *reinterpret_cast<const u32x2*>(ws0 + t * 16 * WROW);
        const u32x2 v1 = *reinterpret_cast<const u32x2*>(ws1 + t * 16 * WROW);
        f.w[t][0] = v0.x;
        f.w[t][1] = v0.y;
        f.w[t][2] = v1.x;
        f.w[t][3] = v1.y;
      }
      if constexpr (TSB) {
        f.sv[t] = *reinterpret_cast<const uint32_t*>(tp + t * 16 * 4);  // (scale, bias)
        f.bv[t] = f.sv[t];
      } else {
        f.sv[t] = *reinterpret_cast<const uint32_t*>(sbp + t * 16 * SBP);
        f.bv[t] = *reinterpret_cast<const uint32_t*>(sbp + t * 16 * SBP + NB * SBP);
      }
    }
  }

  // 16-bit value of a packed pair as fp32; sel moves the wanted half to the
  // high half (bf16: that is the fp32 bit pattern)
  __device__ static inline float half_bf16(uint32_t v, uint32_t sel) {
    return __uint_as_float(__builtin_amdgcn_perm(v, v, sel));
  }
  __device__ static inline float half_of(uint32_t v, uint32_t sel) {
    if constexpr (std::is_same<Tag, BF16>::value) {
      return half_bf16(v, sel);
    } else {
      return Num<Tag>::hi(__builtin_amdgcn_perm(v, v, sel));
    }
  }

  // All-ones MFMA operand held in VGPRs (the empty asm keeps the compiler
  // from rematerialising it from SGPRs before every use).
  __device__ static inline u32x4 ones_operand() {
    u32x4 ones = u32x4{Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2};
    asm volatile("" : "+v"(ones));
    return ones;
  }

  __device__ static inline void compute(const Lane& L, const Frag& f, f32x4 (&acc)[NT][MT],
                                        const DqConst& dq) {
    compute(L, f, acc, dq, u32x4{Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2});
  }

  __device__ static inline void compute(const Lane& L, const Frag& f, f32x4 (&acc)[NT][MT],
                                        const DqConst& dq, const u32x4 ones) {
    // group sums of the slice: lane (col, kg) gets X[m = 4 kg + r] in register r
    f32x4 xs[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (PAIR) {
        xs[mt][0] = Num<Tag>::mma(f.x[mt][1], ones, Num<Tag>::mma(f.x[mt][0], ones, zero4()));
      } else {
        xs[mt][0] = Num<Tag>::mma(f.x[mt][0], ones, zero4());
        xs[mt][1] = Num<Tag>::mma(f.x[mt][1], ones, zero4());
      }
    }
    // Product operands: 4-bit weights take the k-permuted dequantisation
    // (seven VALU operations a word instead of nine), the activations the
    // same permutation (four permutes a fragment, shared by the NT tiles).
    u32x4 xa[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 2; ++j) xa[mt][j] = BITS == 4 ? kperm_x(f.x[mt][j]) : f.x[mt][j];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      u32x4 b0, b1;
      if constexpr (BITS == 4) {
        b0 = dequant_word4_kperm<Tag>(f.w[t][0], dq);
        b1 = dequant_word4_kperm<Tag>(f.w[t][1], dq);
      } else {
        b0 = dequant_word8<Tag>(f.w[t][0], f.w[t][1], dq);
        b1 = dequant_word8<Tag>(f.w[t][2], f.w[t][3], dq);
      }
      if constexpr (PAIR) {
        // window: this wavefront's half of a dword of two groups; TSB: the
        // pair's low (scale) and high (bias) halves
        const float s = half_of(f.sv[t], TSB ? 0x01000c0cu : L.hsel);
        const float bq = __builtin_fmaf(-OFFQ, s, half_of(f.bv[t], TSB ? 0x03020c0cu : L.hsel));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4 p = Num<Tag>::mma(xa[mt][1], b1, Num<Tag>::mma(xa[mt][0], b0, zero4()));
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[t][mt][r] = __builtin_fmaf(bq, xs[mt][0][r], __builtin_fmaf(s, p[r], acc[t][mt][r]));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t sel = j ? 0x03020c0cu : 0x01000c0cu;
          const float s = half_of(f.sv[t], sel);
          const float bq = __builtin_fmaf(-OFFQ, s, half_of(f.bv[t], sel));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f32x4 p = Num<Tag>::mma(xa[mt][j], j ? b1 : b0, zero4());
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[t][mt][r] =
                  __builtin_fmaf(bq, xs[mt][j][r], __builtin_fmaf(s, p[r], acc[t][mt][r]));
          }
        }
      }
    }
  }

  // Bias terms (b - OFF s) X of up to four steps, applied by one fp32 MFMA
  // (16x16x4: D[m][n] += sum over the batch of A[m][slot] B[slot][n])
  // instead of four FMAs per accumulator and step: lane (col, kg) records,
  // for the step in batch slot kg, X of activation row col (A operand) and
  // b - OFF s of weight row col (B operand).  Slots not yet written hold 0.
  // Two k-blocks per group (gs >= 64) only; gs = 32 keeps the FMAs.
  struct Bias {
    float ax[MT];
    float bb[NT];
  };
  __device__ static inline void bias_zero(Bias& z) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) z.ax[mt] = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) z.bb[t] = 0.f;
  }
  __device__ static inline void bias_flush(Bias& z, f32x4 (&acc)[NT][MT]) {
    if constexpr (PAIR) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(z.ax[mt], z.bb[t], acc[t][mt], 0, 0, 0);
      bias_zero(z);
    }
  }

  // compute() with the step's bias terms recorded in z (mine: this lane's kg
  // is the step's batch slot); the caller flushes z after the fourth step of
  // a batch and after the last step of a range.
  __device__ static inline void compute_b(const Lane& L, const Frag& f, f32x4 (&acc)[NT][MT],
                                          const DqConst& dq, const u32x4 ones, Bias& z,
                                          const bool mine) {
    if constexpr (!PAIR) {
      compute(L, f, acc, dq, ones);
    } else {
      // X of activation row col in every register: the ones operand as A,
      // the activation fragment (row col, this lane's k) as B
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const f32x4 xt = Num<Tag>::mma(ones, f.x[mt][1], Num<Tag>::mma(ones, f.x[mt][0], zero4()));
        z.ax[mt] = mine ? xt[0] : z.ax[mt];
      }
      u32x4 xa[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 2; ++j) xa[mt][j] = BITS == 4 ? kperm_x(f.x[mt][j]) : f.x[mt][j];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        u32x4 b0, b1;
        if constexpr (BITS == 4) {
          b0 = dequant_word4_kperm<Tag>(f.w[t][0], dq);
          b1 = dequant_word4_kperm<Tag>(f.w[t][1], dq);
        } else {
          b0 = dequant_word8<Tag>(f.w[t][0], f.w[t][1], dq);
          b1 = dequant_word8<Tag>(f.w[t][2], f.w[t][3], dq);
        }
        const float s = half_of(f.sv[t], TSB ? 0x01000c0cu : L.hsel);
        const float bq = __builtin_fmaf(-OFFQ, s, half_of(f.bv[t], TSB ? 0x03020c0cu : L.hsel));
        z.bb[t] = mine ? bq : z.bb[t];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4 p = Num<Tag>::mma(xa[mt][1], b1, Num<Tag>::mma(xa[mt][0], b0, zero4()));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[t][mt][r] = __builtin_fmaf(s, p[r], acc[t][mt][r]);
        }
      }
    }
  }

  // Barrier once this wavefront has at most n whole steps of loads
  // outstanding (n <= 3).  The scale window precedes every step's loads, so
  // it has landed by the first wait.
  __device__ static inline void wait_steps(int n) {
    if (n >= 3) stage_barrier<3 * CHUNK_DMA>();
    else if (n == 2) stage_barrier<2 * CHUNK_DMA>();
    else if (n == 1) stage_barrier<CHUNK_DMA>();
    else stage_barrier<0>();
  }

  // iteration c: step c+1 must be in LDS (steps c+2 .. c+DEPTH-1 may still
  // be in flight); step c is in `cur`.
  template <bool BM>
  __device__ static inline void step(const Ctx& cx, const Lane& L, int c, int c0, int c1,
                                     int stage, int g0w, Frag& cur, Frag& nxt,
                                     f32x4 (&acc)[NT][MT], const DqConst& dq, const u32x4 ones,
                                     Bias& z) {
    if (c + 1 < c1) {
      wait_steps(min(DEPTH - 2, c1 - c - 2));
      if (c + DEPTH < c1)
        issue_chunk(cx, L, c + DEPTH, stage);  // step c's stage: its fragments are in cur
    }
    // The next step's fragments -- read on the last step too (a stage whose
    // loads have all landed, in bounds, the values unused), so that nxt is
    // always written here and the two fragment sets need no register copies
    // between iterations.  The epilogue's barrier orders these reads before
    // anything reuses the stages.
    const int st1 = stage == DEPTH - 1 ? 0 : stage + 1;
    read_frag(cx, L, c + 1, st1, g0w, nxt);
    if constexpr (BM) {
      const int slot = (c - c0) & 3;  // batch slot of this step's bias terms
      compute_b(L, cur, acc, dq, ones, z, (cx.lane >> 4) == slot);
      if (slot == 3 || c + 1 == c1) bias_flush(z, acc);
    } else {
      compute(L, cur, acc, dq, ones);
    }
  }

  // Accumulate steps [c0, c1) (c1 > c0) of this workgroup into acc.  Every
  // wavefront of the workgroup calls this with the same range (it contains
  // barriers).  The range covers at most MAX_GROUPS groups.  BM: bias terms
  // batched into fp32 MFMAs (compute_b); measured on MI355X faster for the
  // lm_head's long ranges (20 steps per workgroup: 104.6 -> 98.0 us) and
  // slower for the 27B-class sweep's split ranges and the MoE units, which
  // keep the per-step FMAs.
  template <bool BM = false>
  __device__ static inline void run(const Ctx& cx, int c0, int c1, f32x4 (&acc)[NT][MT]) {
    const DqConst dq = dq_const<Tag>();
    const u32x4 ones = ones_operand();
    const Lane L = lane_setup(cx);
    const int piece0 = (c0 * GPC) >> 3;
    const int g0w = piece0 * 8;
    if constexpr (!TSB) issue_sb(cx, piece0, ((c1 * GPC + 7) >> 3) - piece0);
    issue_chunk(cx, L, c0, 0);
#pragma unroll
    for (int k = 1; k < DEPTH; ++k)
      if (c0 + k < c1) issue_chunk(cx, L, c0 + k, k);
    // step c0 in LDS: at most the loads of steps c0+1 .. c0+DEPTH-1 outstanding
    wait_steps(min(DEPTH - 1, c1 - c0 - 1));
    Frag fa, fb;
    read_frag(cx, L, c0, 0, g0w, fa);
    Bias z;
    bias_zero(z);
    int c = c0, stage = 0;
    for (; c + 1 < c1; c += 2) {
      step<BM>(cx, L, c, c0, c1, stage, g0w, fa, fb, acc, dq, ones, z);
      stage = stage == DEPTH - 1 ? 0 : stage + 1;
      step<BM>(cx, L, c + 1, c0, c1, stage, g0w, fb, fa, acc, dq, ones, z);
      stage = stage == DEPTH - 1 ? 0 : stage + 1;
    }
    if (c < c1) step<BM>(cx, L, c, c0, c1, stage, g0w, fa, fb, acc, dq, ones, z);
  }
};

}  // namespace dfmi
