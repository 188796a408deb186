// Streaming main loop of the verify-path matmuls (fast path).
//
// A workgroup of 4 wavefronts owns a block of NB = 64 weight rows (four
// 16-row MFMA tiles) and a range of K chunks (256 k = 128 bytes of every
// int4 weight row).  Cost model (measured on MI355X):
//
//   * a CU's vector memory pipeline retires roughly one cache-line request
//     every few cycles however few bytes of the line an instruction uses, so
//     every global read is a whole-line request: weights (8 rows x 128 B per
//     instruction), activations (2 rows x 512 B) and scales / biases
//     (8 rows x 64 B of each array) go straight to LDS with
//     global_load_lds_dwordx4, kDepth chunks ahead;
//   * LDS read latency is hidden by register double buffering: the fragments
//     of chunk c+1 are read from LDS while chunk c is computed;
//   * each wavefront takes a 64-k slice of every chunk for all four tiles, so
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
// chunk it needs) followed by a workgroup barrier, once per chunk.  The same
// barrier (with lgkmcnt(0)) proves that every wavefront has finished reading
// the stage the next DMA overwrites.
#pragma once

#include "dfmi_core.h"

namespace dfmi {

constexpr int kStreamWaves = 4;
constexpr int kStreamThreads = kStreamWaves * 64;
constexpr int kStreamRows = 64;   // weight rows per workgroup
constexpr int kStreamTiles = 4;   // 16-row MFMA tiles per workgroup, all in every wavefront
constexpr int kDepth = 3;         // LDS stages

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

// Dynamic LDS of the streaming kernels (one allocation per workgroup).
extern __shared__ __attribute__((aligned(16))) char dfmi_smem[];

__device__ inline void dma16(const void* g, void* lds_uniform) {
  __builtin_amdgcn_global_load_lds(const_cast<void*>(g), lds_uniform, 16, 0, 0);
}

template <typename Tag, int GS, int MT>
struct Stream {
  static constexpr int NT = kStreamTiles;
  static constexpr int NB = kStreamRows;
  static constexpr int GPC = kChunkK / GS;  // quantisation groups per chunk
  static constexpr int SBC = 32 / GPC;      // chunks per scale / bias block (32 groups)
  // gs >= 64: a lane's two k-blocks take adjacent words (one 8-byte LDS read);
  // gs = 32: k-block j is group 2*wave + j, so the blocks stay group-pure.
  static constexpr bool PAIR = GS >= 64;
  static constexpr int XBUF = MT * 16 * 512;  // bytes of one activation stage
  static constexpr int WBUF = NB * 128;       // bytes of one weight stage
  static constexpr int SBBUF = NB * 128;      // per row: 64 B of scales, then 64 B of biases
  static constexpr int X_OFF = 0;
  static constexpr int W_OFF = kDepth * XBUF;
  static constexpr int SB_OFF = W_OFF + kDepth * WBUF;
  static constexpr int LDS_BYTES = SB_OFF + 2 * SBBUF;
  // epilogue: [wave][t][mt][reg][lane] floats, aliasing the stages
  static constexpr int RED_FLOATS = NT * MT * 4 * 64;
  static_assert(kStreamWaves * RED_FLOATS * 4 <= LDS_BYTES, "reduction buffer");
  // DMA instructions per wavefront
  static constexpr int X_DMA = MT * 2;  // MT*16 rows x 512 B per stage / 4 waves / 1 KiB
  static constexpr int W_DMA = 2;       // 64 rows x 128 B / 4 waves / 1 KiB
  static constexpr int SB_DMA = 2;      // 64 rows x 128 B per block / 4 waves / 1 KiB
  static constexpr int CHUNK_DMA = X_DMA + W_DMA;
  static_assert(GS == 32 || GS == 64 || GS == 128, "group size");

  struct Ctx {
    const uint16_t* x;
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    int K, M, N;
    int groups;  // K / GS
    int n0;      // first weight row of this workgroup
    int wave, lane;
  };

  // One chunk's operands of this lane, read from LDS.
  struct Frag {
    u32x4 x[MT][2];     // activations of k-block j
    uint32_t w[NT][2];  // packed words of k-block j
    uint32_t sv[NT];    // dword holding this lane's scale(s)
    uint32_t bv[NT];    // dword holding this lane's bias(es)
  };

  // word (= 8-k piece) of the chunk that lane group kg feeds k-block j with
  __device__ static inline int piece_of(int wave, int kg, int j) {
    return PAIR ? 8 * wave + 2 * kg + j : 8 * wave + 4 * j + kg;
  }

  // Activation stage: instruction j covers rows 2j, 2j+1; lane l loads piece
  // (l & 31) ^ (row & 15) of its row into slot l & 31.  Rows >= M re-read
  // row M-1 (their outputs are never stored).
  __device__ static inline void issue_x(const Ctx& cx, int c, int stage) {
#pragma unroll
    for (int i = 0; i < X_DMA; ++i) {
      const int j = cx.wave * X_DMA + i;
      const int r = 2 * j + (cx.lane >> 5);
      const int slot = cx.lane & 31;
      const int piece = slot ^ (r & 15);
      const int m = min(r, cx.M - 1);
      const uint16_t* g = cx.x + (int64_t)m * cx.K + c * kChunkK + piece * 8;
      dma16(g, dfmi_smem + X_OFF + stage * XBUF + j * 1024);
    }
  }

  // Weight stage: instruction i of wavefront w covers rows 8*(2w+i) .. +7;
  // lane l loads piece (l & 7) ^ (row & 7) of its row into slot l & 7.
  // Rows >= N re-read row N-1.
  __device__ static inline void issue_w(const Ctx& cx, int c, int stage) {
    const uint32_t kw = (uint32_t)(cx.K / 8);
#pragma unroll
    for (int i = 0; i < W_DMA; ++i) {
      const int r0 = (cx.wave * W_DMA + i) * 8;
      const int r = r0 + (cx.lane >> 3);
      const int piece = (cx.lane & 7) ^ (r & 7);
      const int n = min(cx.n0 + r, cx.N - 1);
      const uint32_t* g = cx.w + (uint32_t)n * kw + (uint32_t)c * 32u + piece * 4;
      dma16(g, dfmi_smem + W_OFF + stage * WBUF + r0 * 128);
    }
  }

  // Scale / bias block sb = groups [32 sb, 32 sb + 32) of every row: per row
  // 4 pieces of 16 B of each array; lane l of instruction i (rows r0 .. r0+7)
  // loads array (l >> 2) & 1, piece (l & 3) ^ ((row >> 1) & 3) into slot l & 3.
  // Pieces past the end of a row re-read its last piece (never used).
  __device__ static inline void issue_sb(const Ctx& cx, int sb, int buf) {
    const int last_piece = cx.groups / 8 - 1;  // 8 16-bit values per piece
#pragma unroll
    for (int i = 0; i < SB_DMA; ++i) {
      const int r0 = (cx.wave * SB_DMA + i) * 8;
      const int r = r0 + (cx.lane >> 3);
      const int arr = (cx.lane >> 2) & 1;
      const int q = (cx.lane & 3) ^ ((r >> 1) & 3);
      const int n = min(cx.n0 + r, cx.N - 1);
      const int piece = min(sb * 4 + q, last_piece);
      const uint16_t* base = arr ? cx.b : cx.s;
      const uint16_t* g = base + (int64_t)n * cx.groups + piece * 8;
      dma16(g, dfmi_smem + SB_OFF + buf * SBBUF + r0 * 128);
    }
  }

  __device__ static inline void issue_chunk(const Ctx& cx, int c, int stage) {
    issue_x(cx, c, stage);
    issue_w(cx, c, stage);
  }

  // Chunk c's fragments of this lane from LDS stage `stage`, scale buffer sbuf.
  __device__ static inline void read_frag(const Ctx& cx, int c, int stage, int sbuf, Frag& f) {
    const int col = cx.lane & 15, kg = cx.lane >> 4;
    const char* xs = dfmi_smem + X_OFF + stage * XBUF;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + col;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int slot = piece_of(cx.wave, kg, j) ^ col;
        f.x[mt][j] = *reinterpret_cast<const u32x4*>(xs + m * 512 + slot * 16);
      }
    }
    const char* ws = dfmi_smem + W_OFF + stage * WBUF;
    // group index of this lane's first k-block inside the scale / bias block
    const int gi = (c % SBC) * GPC + (PAIR ? (cx.wave * 64) / GS : 2 * cx.wave);
    const int sbyte = gi * 2;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int r = t * 16 + col;
      const char* row = ws + r * 128;
      if constexpr (PAIR) {
        const int byte = piece_of(cx.wave, kg, 0) * 4;
        const int slot = (byte >> 4) ^ (r & 7);
        const u32x2 v = *reinterpret_cast<const u32x2*>(row + slot * 16 + (byte & 15));
        f.w[t][0] = v.x;
        f.w[t][1] = v.y;
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int byte = piece_of(cx.wave, kg, j) * 4;
          const int slot = (byte >> 4) ^ (r & 7);
          f.w[t][j] = *reinterpret_cast<const uint32_t*>(row + slot * 16 + (byte & 15));
        }
      }
      const int slot = (sbyte >> 4) ^ ((r >> 1) & 3);
      const char* p = dfmi_smem + SB_OFF + sbuf * SBBUF + r * 128 + slot * 16 + (sbyte & 12);
      f.sv[t] = *reinterpret_cast<const uint32_t*>(p);
      f.bv[t] = *reinterpret_cast<const uint32_t*>(p + 64);
    }
  }

  // 16-bit value (half 0: low, 1: high) of a packed pair as fp32
  __device__ static inline float half_of(uint32_t v, int half) {
    return half ? Num<Tag>::hi(v) : Num<Tag>::lo(v);
  }

  __device__ static inline void compute(const Ctx& cx, const Frag& f, f32x4 (&acc)[NT][MT],
                                        const DqConst& dq) {
    const u32x4 ones = u32x4{Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2};
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
    // which half of the scale dword is this wavefront's group (gs >= 64)
    const int half = PAIR ? (((cx.wave * 64) / GS) & 1) : 0;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const u32x4 b0 = dequant_word4<Tag>(f.w[t][0], dq);
      const u32x4 b1 = dequant_word4<Tag>(f.w[t][1], dq);
      if constexpr (PAIR) {
        const float s = half_of(f.sv[t], half);
        const float bq = __builtin_fmaf(-Num<Tag>::OFF, s, half_of(f.bv[t], half));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4 p = Num<Tag>::mma(f.x[mt][1], b1, Num<Tag>::mma(f.x[mt][0], b0, zero4()));
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[t][mt][r] = __builtin_fmaf(bq, xs[mt][0][r], __builtin_fmaf(s, p[r], acc[t][mt][r]));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float s = half_of(f.sv[t], j);
          const float bq = __builtin_fmaf(-Num<Tag>::OFF, s, half_of(f.bv[t], j));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f32x4 p = Num<Tag>::mma(f.x[mt][j], j ? b1 : b0, zero4());
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[t][mt][r] =
                  __builtin_fmaf(bq, xs[mt][j][r], __builtin_fmaf(s, p[r], acc[t][mt][r]));
          }
        }
      }
    }
  }

  // Wait for the loads of one chunk: n = loads this wavefront issued after
  // them (one of 0, C, C+S, 2C, 2C+S with C = CHUNK_DMA, S = SB_DMA).
  __device__ static inline void wait_chunk(int n) {
    constexpr int C = CHUNK_DMA, S = SB_DMA;
    if (n == C) stage_barrier<C>();
    else if (n == C + S) stage_barrier<C + S>();
    else if (n == 2 * C) stage_barrier<2 * C>();
    else if (n == 2 * C + S) stage_barrier<2 * C + S>();
    else stage_barrier<0>();
  }

  // loads issued for chunk c (0 when c is past the range end c1)
  __device__ static inline int loads_of(int c, int c1) {
    return c < c1 ? CHUNK_DMA + ((c % SBC) == 0 ? SB_DMA : 0) : 0;
  }

  // iteration c: chunk c+1 must be in LDS; chunk c is in `cur`
  __device__ static inline void step(const Ctx& cx, int c, int c1, int stage, Frag& cur,
                                     Frag& nxt, f32x4 (&acc)[NT][MT], const DqConst& dq) {
    if (c + 1 < c1) {
      wait_chunk(loads_of(c + 2, c1));
      if (c + 3 < c1) {
        if ((c + 3) % SBC == 0) issue_sb(cx, (c + 3) / SBC, ((c + 3) / SBC) & 1);
        issue_chunk(cx, c + 3, stage);  // chunk c's stage: its fragments are in cur
      }
      const int st1 = stage == 2 ? 0 : stage + 1;
      read_frag(cx, c + 1, st1, ((c + 1) / SBC) & 1, nxt);
    }
    compute(cx, cur, acc, dq);
  }

  // Accumulate chunks [c0, c1) (c1 > c0) of this workgroup into acc.  Every
  // wavefront of the workgroup calls this with the same range (it contains
  // barriers).
  __device__ static inline void run(const Ctx& cx, int c0, int c1, f32x4 (&acc)[NT][MT]) {
    const DqConst dq = dq_const<Tag>();
    issue_sb(cx, c0 / SBC, (c0 / SBC) & 1);
    issue_chunk(cx, c0, 0);
#pragma unroll
    for (int k = 1; k < kDepth; ++k) {
      if (c0 + k < c1) {
        if ((c0 + k) % SBC == 0) issue_sb(cx, (c0 + k) / SBC, ((c0 + k) / SBC) & 1);
        issue_chunk(cx, c0 + k, k);
      }
    }
    wait_chunk(loads_of(c0 + 1, c1) + loads_of(c0 + 2, c1));
    Frag fa, fb;
    read_frag(cx, c0, 0, (c0 / SBC) & 1, fa);
    int c = c0, stage = 0;
    for (; c + 1 < c1; c += 2) {
      step(cx, c, c1, stage, fa, fb, acc, dq);
      stage = stage == 2 ? 0 : stage + 1;
      step(cx, c + 1, c1, stage, fb, fa, acc, dq);
      stage = stage == 2 ? 0 : stage + 1;
    }
    if (c < c1) step(cx, c, c1, stage, fa, fb, acc, dq);
  }
};

}  // namespace dfmi
