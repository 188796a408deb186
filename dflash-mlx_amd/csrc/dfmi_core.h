// Main loop of every verify-path matmul.
//
// A workgroup owns NT 16-row weight tiles (16*NT output columns) and all M
// rows of the activations (MT 16-row MFMA blocks).  Its W wavefronts split K:
// wavefront w streams its share of the K "chunks" (256 k = 128 bytes of each
// int4 weight row) for all NT tiles, and the W partial tiles are summed once
// through LDS at the end.  There is no cross-workgroup reduction, hence no
// device-scope fence and no atomic on the matmul path.
//
// Per chunk and wavefront lane (col = lane & 15, kg = lane >> 4):
//   * weights: for each group g of the chunk the lane loads the WPL = gs/32
//     consecutive words kg*WPL .. of that group (one dword / dwordx2 / dwordx4
//     load), so the 4 lanes of one column cover the group and every
//     16x16x32 MFMA stays inside one quantisation group;
//   * activations: the 8 fragments (16 rows x 256 k) straight from global
//     memory (L2-resident: every workgroup reads the same x), used as MFMA
//     operands in k order (dequant_word4 emits the weights in k order);
//   * X[m, g] (group sums of the activations) come from MFMAs against an
//     all-ones operand, which lands them in the layout the fp32 bias MFMA needs.
// Chunk c+1 is loaded (unconditionally: the index is clamped to the last
// chunk, whose lines are then already in cache) before chunk c is computed,
// so every wait in the loop is for loads issued one iteration earlier.
#pragma once

#include "dfmi_device.h"

namespace dfmi {

constexpr int kMaxWaves = 8;
constexpr int kChunkK = 256;

template <typename Tag, int GS, int MT, int NT, bool KFULL>
struct Core {
  static constexpr int GPC = kChunkK / GS;     // quantisation groups per chunk (8/4/2)
  static constexpr int WPL = GS / 32;          // words per lane per group (1/2/4)
  static constexpr int FR = kChunkK / 32;      // 16x16x32 MFMA k-blocks per chunk (8)
  static constexpr int NBB = (GPC + 3) / 4;    // fp32 bias MFMAs per chunk and tile
  static constexpr int SVEC = (GPC + 1) / 2;   // u32 registers for the chunk's scales
  // LDS for the cross-wavefront reduction: [wave][t][mt][reg][lane] floats.
  static constexpr int RED_FLOATS_PER_WAVE = NT * MT * 4 * 64;
  static constexpr int LDS_BYTES = kMaxWaves * RED_FLOATS_PER_WAVE * 4;
  static_assert(GS == 32 || GS == 64 || GS == 128, "group size");

  struct Tile {
    uint32_t w[FR];    // packed words, group g word h at w[g*WPL + h]
    uint32_t s[SVEC];  // the chunk's GPC scales of this lane's row, packed pairs
    uint32_t b[SVEC];  // the chunk's GPC biases of this lane's row, packed pairs
  };

  struct XFrag {
    u32x4 v[MT][FR];  // activations of the chunk, fragment f = MFMA k-block f
  };

  // Per-tile row addressing of this lane.
  struct Rows {
    const uint32_t* wbase[NT];
    const uint16_t* sbase[NT];
    const uint16_t* bbase[NT];
    uint32_t woff[NT];  // word offset of this lane's row in tile t
    uint32_t soff[NT];  // element offset of this lane's row in scales / biases
  };

  // Activation rows of this lane: element offset of row mt*16 + (lane&15).
  // Rows >= M point at a valid row instead: MFMA rows are independent, so a
  // duplicated activation row only produces output rows that are never
  // stored, and every load stays unconditional (a load under a divergent
  // branch would force the compiler to wait for all outstanding loads).
  struct XRows {
    int64_t off[MT];
  };

  __device__ static inline XRows x_rows(int m_base, int M, int K, int lane) {
    XRows xr;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = min(m_base + mt * 16 + (lane & 15), M - 1);
      xr.off[mt] = (int64_t)m * K;
    }
    return xr;
  }

  __device__ static inline void load_x(XFrag& xf, const uint16_t* __restrict__ x,
                                       const XRows& xr, int c, int K, int kg) {
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      const int g = f / WPL, h = f % WPL;
      const int k = c * kChunkK + g * GS + (kg * WPL + h) * 8;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (KFULL || k < K) {
          xf.v[mt][f] = *reinterpret_cast<const u32x4*>(x + xr.off[mt] + k);
        } else {
          xf.v[mt][f] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  }

  __device__ static inline void load_tile(Tile& t, const uint32_t* __restrict__ wbase,
                                          const uint16_t* __restrict__ sbase,
                                          const uint16_t* __restrict__ bbase, uint32_t woff,
                                          uint32_t soff, int c, int K, int kg) {
    const uint32_t* wp = wbase + woff + (uint32_t)c * 32u + (uint32_t)(kg * WPL);
#pragma unroll
    for (int g = 0; g < GPC; ++g) {
      const bool ok = KFULL || (c * kChunkK + g * GS) < K;
      if constexpr (WPL == 1) {
        t.w[g] = ok ? wp[g * 4] : 0u;
      } else if constexpr (WPL == 2) {
        u32x2 v = ok ? *reinterpret_cast<const u32x2*>(wp + g * 8) : u32x2{0u, 0u};
        t.w[2 * g] = v.x;
        t.w[2 * g + 1] = v.y;
      } else {
        u32x4 v = ok ? *reinterpret_cast<const u32x4*>(wp + g * 16) : u32x4{0u, 0u, 0u, 0u};
        t.w[4 * g] = v.x;
        t.w[4 * g + 1] = v.y;
        t.w[4 * g + 2] = v.z;
        t.w[4 * g + 3] = v.w;
      }
    }
    const uint32_t so = soff + (uint32_t)(c * GPC);
    if constexpr (KFULL) {
      load_vec(t.s, sbase + so);
      load_vec(t.b, bbase + so);
    } else {
#pragma unroll
      for (int j = 0; j < SVEC; ++j) {
        uint32_t slo = 0u, shi = 0u, blo = 0u, bhi = 0u;
        if ((c * kChunkK + (2 * j) * GS) < K) {
          slo = sbase[so + 2 * j];
          blo = bbase[so + 2 * j];
        }
        if (2 * j + 1 < GPC && (c * kChunkK + (2 * j + 1) * GS) < K) {
          shi = sbase[so + 2 * j + 1];
          bhi = bbase[so + 2 * j + 1];
        }
        t.s[j] = slo | (shi << 16);
        t.b[j] = blo | (bhi << 16);
      }
    }
  }

  // The chunk's GPC 16-bit values of one row (scales or biases) in SVEC registers.
  __device__ static inline void load_vec(uint32_t (&dst)[SVEC], const uint16_t* __restrict__ p) {
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(p);
    if constexpr (SVEC == 4) {
      u32x4 v = *reinterpret_cast<const u32x4*>(sp);
      dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    } else if constexpr (SVEC == 2) {
      u32x2 v = *reinterpret_cast<const u32x2*>(sp);
      dst[0] = v.x; dst[1] = v.y;
    } else {
      dst[0] = sp[0];
    }
  }

  // 16-bit value of group 4*bb + kg (0 when the chunk has no such group).
  // Bitwise selects only: a lane-dependent array index would be lowered to a
  // scratch-memory round trip.
  __device__ static inline uint32_t lane_group_value(const uint32_t (&v)[SVEC], int bb, int kg) {
    uint32_t reg;
    if constexpr (SVEC == 1) {
      reg = v[0];
    } else {
      const uint32_t hi_mask = 0u - (uint32_t)((kg >> 1) & 1);
      reg = (v[2 * bb + 1] & hi_mask) | (v[2 * bb] & ~hi_mask);
    }
    const uint32_t val = (reg >> ((kg & 1) * 16)) & 0xFFFFu;
    return (4 * bb + kg < GPC) ? val : 0u;
  }

  __device__ static inline void load_chunk(XFrag& xf, Tile (&tl)[NT], const uint16_t* __restrict__ x,
                                           const XRows& xr, const Rows& r, int c, int K, int kg) {
    load_x(xf, x, xr, c, K, kg);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      load_tile(tl[t], r.wbase[t], r.sbase[t], r.bbase[t], r.woff[t], r.soff[t], c, K, kg);
  }

  __device__ static inline float scale_of(const Tile& t, int g) {
    return (g & 1) ? Num<Tag>::hi(t.s[g >> 1]) : Num<Tag>::lo(t.s[g >> 1]);
  }

  __device__ static inline void compute_chunk(const XFrag& xf, const Tile (&tl)[NT],
                                              f32x4 (&acc)[NT][MT], int kg, const DqConst& dq) {
    const auto& a = xf.v;
    // Group sums of the activations: C = ONES . A^T puts X[m = lane&15, g] in every register.
    const u32x4 ones = u32x4{Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2};
    float xa[MT][NBB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float xs[GPC];
#pragma unroll
      for (int g = 0; g < GPC; ++g) {
        f32x4 t = zero4();
#pragma unroll
        for (int h = 0; h < WPL; ++h) t = Num<Tag>::mma(ones, a[mt][g * WPL + h], t);
        xs[g] = t.x;
      }
#pragma unroll
      for (int bb = 0; bb < NBB; ++bb) {
        float v = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (4 * bb + j < GPC) v = (kg == j) ? xs[4 * bb + j] : v;
        }
        xa[mt][bb] = v;
      }
    }

#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int g = 0; g < GPC; ++g) {
        f32x4 p[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) p[mt] = zero4();
#pragma unroll
        for (int h = 0; h < WPL; ++h) {
          const u32x4 b = dequant_word4<Tag>(tl[t].w[g * WPL + h], dq);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) p[mt] = Num<Tag>::mma(a[mt][g * WPL + h], b, p[mt]);
        }
        const float sg = scale_of(tl[t], g);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[t][mt].x = __builtin_fmaf(sg, p[mt].x, acc[t][mt].x);
          acc[t][mt].y = __builtin_fmaf(sg, p[mt].y, acc[t][mt].y);
          acc[t][mt].z = __builtin_fmaf(sg, p[mt].z, acc[t][mt].z);
          acc[t][mt].w = __builtin_fmaf(sg, p[mt].w, acc[t][mt].w);
        }
      }
#pragma unroll
      for (int bb = 0; bb < NBB; ++bb) {
        const float bq =
            __builtin_fmaf(-Num<Tag>::OFF, Num<Tag>::h2f(lane_group_value(tl[t].s, bb, kg)),
                           Num<Tag>::h2f(lane_group_value(tl[t].b, bb, kg)));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mma_f32_16x16x4(xa[mt][bb], bq, acc[t][mt]);
      }
    }
  }

  // Accumulate chunks [c0, c1) (c1 > c0) into acc (acc is not cleared here).
  //
  // Two register sets A/B; chunk c+1 is in flight while chunk c is computed.
  // Only valid chunks are ever loaded (a redundant load would add a full
  // memory round trip before the wavefront can retire), and every load sits
  // in straight-line code: the steady-state loop runs while both of its
  // prefetches are valid and the last two or three chunks are peeled, so the
  // compiler can wait for exactly the older loads (a load behind a branch
  // would make it wait for all of them, or sink the load into the branch).
  // sched_barrier keeps the machine scheduler from sinking a prefetch below
  // the compute it is meant to overlap.
  __device__ static inline void run(const uint16_t* __restrict__ x, const XRows& xr,
                                    const Rows& r, int K, int c0, int c1,
                                    f32x4 (&acc)[NT][MT]) {
    const int kg = (threadIdx.x & 63) >> 4;
    const DqConst dq = dq_const<Tag>();
    if constexpr (MT * NT > 1) {
      // Larger register tiles: a single register set (two would spill).
      for (int c = c0; c < c1; ++c) {
        XFrag xf;
        Tile tl[NT];
        load_chunk(xf, tl, x, xr, r, c, K, kg);
        compute_chunk(xf, tl, acc, kg, dq);
      }
      return;
    }
    XFrag xa, xb;
    Tile ta[NT], tb[NT];
    load_chunk(xa, ta, x, xr, r, c0, K, kg);
    if (c1 - c0 == 1) {
      compute_chunk(xa, ta, acc, kg, dq);
      return;
    }
    load_chunk(xb, tb, x, xr, r, c0 + 1, K, kg);
    __builtin_amdgcn_sched_barrier(0);
    int c = c0;
    for (; c + 3 < c1; c += 2) {
      compute_chunk(xa, ta, acc, kg, dq);
      load_chunk(xa, ta, x, xr, r, c + 2, K, kg);
      __builtin_amdgcn_sched_barrier(0);
      compute_chunk(xb, tb, acc, kg, dq);
      load_chunk(xb, tb, x, xr, r, c + 3, K, kg);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c1 - c == 3) {
      compute_chunk(xa, ta, acc, kg, dq);
      load_chunk(xa, ta, x, xr, r, c + 2, K, kg);
      __builtin_amdgcn_sched_barrier(0);
      compute_chunk(xb, tb, acc, kg, dq);
      compute_chunk(xa, ta, acc, kg, dq);
    } else {
      compute_chunk(xa, ta, acc, kg, dq);
      compute_chunk(xb, tb, acc, kg, dq);
    }
  }

  // Sum the wavefronts' partial tiles through LDS; afterwards thread e
  // (e < RED_FLOATS_PER_WAVE, e = ((t*MT + mt)*4 + reg)*64 + lane) calls
  // out(t, mt, reg, lane, value) for each element it owns.
  template <typename Out>
  __device__ static inline void reduce(float* lds, const f32x4 (&acc)[NT][MT], int waves,
                                       Out&& out) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* mine = lds + wave * RED_FLOATS_PER_WAVE;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) mine[((t * MT + mt) * 4 + j) * 64 + lane] = acc[t][mt][j];
    __syncthreads();
    for (int e = tid; e < RED_FLOATS_PER_WAVE; e += waves * 64) {
      float s = lds[e];
      for (int w = 1; w < waves; ++w) s += lds[w * RED_FLOATS_PER_WAVE + e];
      const int l = e & 63, j = (e >> 6) & 3, tm = e >> 8;
      out(tm / MT, tm % MT, j, l, s);
    }
  }
};

}  // namespace dfmi
