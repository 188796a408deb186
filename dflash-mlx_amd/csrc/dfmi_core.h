// Main loop of every verify-path matmul: a workgroup of 4 wavefronts streams
// the packed weights of 4*NT 16-row tiles over a range of K "chunks" (256 k
// = 128 bytes of each int4 weight row), with the activations for the chunk
// staged once per workgroup in LDS.
//
// Per chunk and wavefront lane (col = lane & 15, kg = lane >> 4):
//   * weights: for each group g of the chunk the lane loads the WPL = gs/32
//     consecutive words kg*WPL .. of that group (one dword / dwordx2 / dwordx4
//     load), so the 4 lanes of one column cover the group and every
//     16x16x32 MFMA stays inside one quantisation group;
//   * the 8 activation fragments (16 rows x 256 k, pre-permuted to the
//     nibble order of dequant_word4) come from LDS with ds_read_b128;
//   * X[m, g] (group sums of the activations) come from MFMAs against an
//     all-ones operand, which lands them in the layout the fp32 bias MFMA needs.
// The next chunk's weights and activations are in flight while the current
// one is computed (two register sets, two LDS buffers, one barrier per chunk).
#pragma once

#include "dfmi_device.h"

namespace dfmi {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kChunkK = 256;

template <typename Tag, int GS, int MT, int NT, bool KFULL>
struct Core {
  static constexpr int GPC = kChunkK / GS;     // quantisation groups per chunk (8/4/2)
  static constexpr int WPL = GS / 32;          // words per lane per group (1/2/4)
  static constexpr int FR = kChunkK / 32;      // 16x16x32 MFMA k-blocks per chunk (8)
  static constexpr int NBB = (GPC + 3) / 4;    // fp32 bias MFMAs per chunk and tile
  static constexpr int SPT = MT * FR * 64 / kThreads;  // staging slots per thread
  static constexpr int SVEC = (GPC + 1) / 2;   // u32 registers for the chunk's scales
  static constexpr int LDS_BUF = MT * FR * 64 * 16;    // bytes of one staged chunk
  static constexpr int LDS_BYTES = 2 * LDS_BUF;
  static_assert(GS == 32 || GS == 64 || GS == 128, "group size");
  static_assert(SPT >= 1, "staging");

  struct Tile {
    uint32_t w[FR];    // packed words, group g word h at w[g*WPL + h]
    uint32_t s[SVEC];  // the chunk's GPC scales of this lane's row, packed pairs
    uint32_t bq[NBB];  // raw 16-bit bias of group 4*bb + kg
    uint32_t sq[NBB];  // raw 16-bit scale of group 4*bb + kg
  };

  // Per-thread staging description (fixed for the whole workgroup).
  struct Stage {
    int64_t xoff[SPT];  // element offset of the activation row start, -1 = zero row
    int kk[SPT];        // k offset of the slot inside a chunk
    int lds[SPT];       // byte offset of the slot inside a buffer
  };

  // Slot s (tid + 256*i) -> (mt, f, l) with MFMA fragment f of row block mt for
  // lane l; row m = mt*16 + (l & 15); k offset g*GS + ((l>>4)*WPL + h)*8.
  __device__ static inline void slot_geometry(int slot, int& m, int& kk) {
    const int mt = slot / (FR * 64);
    const int f = (slot / 64) % FR;
    const int l = slot % 64;
    const int g = f / WPL, h = f % WPL;
    m = mt * 16 + (l & 15);
    kk = g * GS + ((l >> 4) * WPL + h) * 8;
  }

  __device__ static inline void stage_load(const uint16_t* __restrict__ x, const Stage& st, int c,
                                           int K, u32x4 (&v)[SPT]) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int k = c * kChunkK + st.kk[i];
      if (st.xoff[i] >= 0 && (KFULL || k < K)) {
        v[i] = *reinterpret_cast<const u32x4*>(x + st.xoff[i] + k);
      } else {
        v[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  __device__ static inline void stage_store(char* lds_buf, const Stage& st, const u32x4 (&v)[SPT]) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      *reinterpret_cast<u32x4*>(lds_buf + st.lds[i]) = permute_x8(v[i]);
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
      const uint32_t* sp = reinterpret_cast<const uint32_t*>(sbase + so);
      if constexpr (SVEC == 4) {
        u32x4 v = *reinterpret_cast<const u32x4*>(sp);
        t.s[0] = v.x; t.s[1] = v.y; t.s[2] = v.z; t.s[3] = v.w;
      } else if constexpr (SVEC == 2) {
        u32x2 v = *reinterpret_cast<const u32x2*>(sp);
        t.s[0] = v.x; t.s[1] = v.y;
      } else {
        t.s[0] = sp[0];
      }
    } else {
#pragma unroll
      for (int j = 0; j < SVEC; ++j) {
        uint32_t lo = 0u, hi = 0u;
        if ((c * kChunkK + (2 * j) * GS) < K) lo = sbase[so + 2 * j];
        if (2 * j + 1 < GPC && (c * kChunkK + (2 * j + 1) * GS) < K) hi = sbase[so + 2 * j + 1];
        t.s[j] = lo | (hi << 16);
      }
    }
#pragma unroll
    for (int bb = 0; bb < NBB; ++bb) {
      const int gi = 4 * bb + kg;
      const bool ok = gi < GPC && (KFULL || (c * kChunkK + gi * GS) < K);
      t.bq[bb] = ok ? (uint32_t)bbase[so + gi] : 0u;
      t.sq[bb] = ok ? (uint32_t)sbase[so + gi] : 0u;
    }
  }

  __device__ static inline float scale_of(const Tile& t, int g) {
    return (g & 1) ? Num<Tag>::hi(t.s[g >> 1]) : Num<Tag>::lo(t.s[g >> 1]);
  }

  // One chunk: activations from LDS, then every tile of this wavefront.
  __device__ static inline void compute_chunk(const char* lds_buf, const Tile (&tl)[NT],
                                              f32x4 (&acc)[NT][MT], int lane) {
    const int kg = lane >> 4;
    u32x4 a[MT][FR];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int f = 0; f < FR; ++f)
        a[mt][f] = *reinterpret_cast<const u32x4*>(lds_buf + ((mt * FR + f) * 64 + lane) * 16);

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
          const u32x4 b = dequant_word4<Tag>(tl[t].w[g * WPL + h]);
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
        const float bq = __builtin_fmaf(-Num<Tag>::OFF, Num<Tag>::h2f(tl[t].sq[bb]),
                                        Num<Tag>::h2f(tl[t].bq[bb]));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mma_f32_16x16x4(xa[mt][bb], bq, acc[t][mt]);
      }
    }
  }

  struct Rows {
    const uint32_t* wbase[NT];
    const uint16_t* sbase[NT];
    const uint16_t* bbase[NT];
    uint32_t woff[NT];  // word offset of this lane's row in tile t
    uint32_t soff[NT];  // element offset of this lane's row in scales / biases
  };

  __device__ static inline void load_tiles(Tile (&tl)[NT], const Rows& r, int c, int K, int kg) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
      load_tile(tl[t], r.wbase[t], r.sbase[t], r.bbase[t], r.woff[t], r.soff[t], c, K, kg);
  }

  __device__ static inline void step(const uint16_t* __restrict__ x, const Stage& st, const Rows& r,
                                     int c, int c_end, int K, char* lds, int buf,
                                     Tile (&cur)[NT], Tile (&nxt)[NT], f32x4 (&acc)[NT][MT],
                                     int lane) {
    __syncthreads();
    const bool more = (c + 1) < c_end;
    u32x4 xv[SPT];
    if (more) {
      stage_load(x, st, c + 1, K, xv);
      load_tiles(nxt, r, c + 1, K, lane >> 4);
    }
    compute_chunk(lds + buf * LDS_BUF, cur, acc, lane);
    if (more) stage_store(lds + (buf ^ 1) * LDS_BUF, st, xv);
  }

  // Accumulate chunks [c_begin, c_end) into acc (acc is not cleared here).
  __device__ static inline void run(const uint16_t* __restrict__ x, const Stage& st, const Rows& r,
                                    int K, int c_begin, int c_end, char* lds,
                                    f32x4 (&acc)[NT][MT]) {
    const int lane = threadIdx.x & 63;
    Tile ta[NT], tb[NT];
    {
      u32x4 xv[SPT];
      stage_load(x, st, c_begin, K, xv);
      load_tiles(ta, r, c_begin, K, lane >> 4);
      stage_store(lds, st, xv);
    }
    for (int c = c_begin; c < c_end; c += 2) {
      step(x, st, r, c, c_end, K, lds, 0, ta, tb, acc, lane);
      if (c + 1 < c_end) step(x, st, r, c + 1, c_end, K, lds, 1, tb, ta, acc, lane);
    }
  }
};

}  // namespace dfmi
