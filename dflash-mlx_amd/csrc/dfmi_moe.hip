// Routed-expert (MoE) matmuls on gfx950: gather_qmm, the fused SwiGLU front
// half of a SwitchGLU block, and the weighted top-k combine.
//
// Pairs p < P map (activation row lhs_rows[p], expert rhs_experts[p]).  A run
// is a maximal stretch of consecutive pairs with the same expert (after the
// sort mlx-lm's SwitchGLU applies for >= 64 pairs, every expert is one run;
// unsorted pairs just make shorter runs).  Grid: (column blocks, P); the
// workgroup of the first pair of a run streams that expert's weight rows once
// for the whole run, 16 gathered activation rows per MFMA block, and the
// other pairs' workgroups exit at once.
//
//  * gather_stream_kernel (K >= 1024, a multiple of 256 and of 8 groups): the
//    streaming main loop (LDS-DMA staging of whole weight lines, 4
//    wavefronts) over a 64-row block: 64 rows of one expert, or for the fused
//    SwiGLU 32 gate rows and the same 32 up rows, so one workgroup produces
//    32 finished h columns.  The activation DMA takes its rows from lhs_rows.
//  * gather_kernel (every other shape): the general main loop (Core:
//    wavefronts split K, partial tiles summed through LDS), with the
//    activation row of each MFMA lane taken from lhs_rows.
#include <algorithm>
#include <cmath>

#include "dfmi_core.h"
#include "dfmi_host.h"
#include "dfmi_stream.h"

namespace dfmi {

struct GatherArgs {
  const uint16_t* x;
  int64_t x_rows;
  const uint32_t* w[2];  // [0]: the matmul's (or gate) weights, [1]: up weights (SwiGLU)
  const uint16_t* s[2];
  const uint16_t* b[2];
  const int32_t* lhs;    // NULL: row p for pair p
  const int32_t* rhs;
  const uint32_t* t;     // (scale, bias) pair tables [E][K/GS][N or 2N] (moe_stream_kernel)
  uint32_t* ws_counters;  // moe_stream_kernel tail split: counters (zero between calls), or NULL
  float* ws_partials;     // and the pieces' fp32 partial tiles
  uint16_t* y;           // [P, N]
  int P, K, N, E;
  int chunks;
};

template <typename Tag>
__device__ inline float rnd(float v) {
  return Num<Tag>::h2f(Num<Tag>::f2h(v));
}

// silu(g) * u with every op rounded to the activation dtype, as the
// op-by-op MLX sequence sigmoid(g) -> g * sig -> * u does.
template <typename Tag>
__device__ inline float silu_mul(float g, float u) {
  const float sig = rnd<Tag>(1.0f / (1.0f + __expf(-g)));
  const float si = rnd<Tag>(g * sig);
  return si * u;
}

template <typename Tag, int GS, int NT, bool KFULL, bool GLU>
__global__ __launch_bounds__(kMaxWaves * 64) void gather_kernel(GatherArgs a) {
  constexpr int TT = GLU ? 2 * NT : NT;  // Core tiles: the NT gate tiles, then NT up tiles
  using C = Core<Tag, GS, 1, TT, KFULL>;
  __shared__ __attribute__((aligned(16))) float lds[C::LDS_BYTES / 4];

  const int p = blockIdx.y;
  const int e = a.rhs[p];
  if (p > 0 && a.rhs[p - 1] == e) return;  // not the first pair of its run (uniform)
  int run = 1;
  while (p + run < a.P && a.rhs[p + run] == e) ++run;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  const bool bad_e = e < 0 || e >= a.E;
  const int ee = bad_e ? 0 : e;
  const uint32_t kw = (uint32_t)(a.K / 8);
  const uint32_t kgrp = (uint32_t)(a.K / GS);

  typename C::Rows r;
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int which = (GLU && t >= NT) ? 1 : 0;
    const int tt = t % NT;
    const int row = min(n0 + tt * 16 + (lane & 15), a.N - 1);
    r.wbase[t] = a.w[which] + (size_t)ee * a.N * kw;
    r.sbase[t] = a.s[which] + (size_t)ee * a.N * kgrp;
    r.bbase[t] = a.b[which] + (size_t)ee * a.N * kgrp;
    r.woff[t] = (uint32_t)row * kw;
    r.soff[t] = (uint32_t)row * kgrp;
  }

  for (int g0 = 0; g0 < run; g0 += 16) {
    const int rows = min(16, run - g0);
    // activation row of this lane's MFMA row (rows past the run repeat the last pair)
    const int pl = p + g0 + min(lane & 15, rows - 1);
    int xr_row = a.lhs ? a.lhs[pl] : pl;
    if (xr_row < 0 || xr_row >= a.x_rows) xr_row = 0;  // reported as NaN below
    typename C::XRows xr;
    xr.off[0] = (int64_t)xr_row * a.K;

    f32x4 acc[TT][1];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t][0] = zero4();
    if (!bad_e) {
      const int per = (a.chunks + waves - 1) / waves;
      const int c0 = min(wave * per, a.chunks), c1 = min(c0 + per, a.chunks);
      if (c1 > c0) C::run(a.x, xr, r, a.K, c0, c1, acc);
    }

    // sum the wavefronts' partial tiles; element e of tile t < NT (and its up
    // partner at t + NT) -> output (pair p + g0 + m, column n)
    float* mine = lds + wave * C::RED_FLOATS_PER_WAVE;
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) mine[(t * 4 + j) * 64 + lane] = acc[t][0][j];
    __syncthreads();
    constexpr int OUT = NT * 4 * 64;
    for (int el = tid; el < OUT; el += waves * 64) {
      float v = 0.f, u = 0.f;
      for (int w = 0; w < waves; ++w) {
        v += lds[w * C::RED_FLOATS_PER_WAVE + el];
        if (GLU) u += lds[w * C::RED_FLOATS_PER_WAVE + OUT + el];
      }
      const int l = el & 63, j = (el >> 6) & 3, t = el >> 8;
      const int m = 4 * (l >> 4) + j;
      const int n = n0 + t * 16 + (l & 15);
      if (m < rows && n < a.N) {
        const int pp = p + g0 + m;
        const int xrow = a.lhs ? a.lhs[pp] : pp;
        float out;
        if (bad_e || xrow < 0 || xrow >= a.x_rows) {
          out = __builtin_nanf("");
        } else if (GLU) {
          out = silu_mul<Tag>(rnd<Tag>(v), rnd<Tag>(u));
        } else {
          out = v;
        }
        a.y[(int64_t)pp * a.N + n] = Num<Tag>::f2h(out);
      }
    }
    __syncthreads();  // the next group reuses the reduction buffer
  }
}

template <typename Tag, int GS, bool GLU, int SBPC>
__global__ __launch_bounds__(256) void gather_stream_kernel(GatherArgs a) {
  using S = Stream<Tag, GS, 1, 4, SBPC>;
  constexpr int OUTC = GLU ? S::NB / 2 : S::NB;  // output columns per workgroup
  __shared__ int32_t s_rows[16];   // activation row of each MFMA row (clamped)
  __shared__ int32_t s_lhs[16];    // raw lhs ids of the current 16 pairs
  __shared__ int32_t s_rhs[18];    // rhs[p-1 .. p+16]
  const int p = blockIdx.y;
  const int tid = threadIdx.x;
  // One memory round trip for all the indexing: the expert ids around p and
  // the activation rows of the first 16 pairs, loaded together.
  if (tid < 18) {
    const int q = p - 1 + tid;
    s_rhs[tid] = (q >= 0 && q < a.P) ? a.rhs[q] : 0;
  } else if (tid >= 64 && tid < 80) {
    const int q = min(p + tid - 64, a.P - 1);
    s_lhs[tid - 64] = a.lhs ? a.lhs[q] : q;
  }
  __syncthreads();
  const int e = s_rhs[1];
  if (p > 0 && s_rhs[0] == e) return;  // not the first pair of its run (uniform)
  int run = 1;
  while (p + run < a.P && run < 17 && s_rhs[1 + run] == e) ++run;
  if (run == 17)  // a run longer than the window: rare, continue in memory
    while (p + run < a.P && a.rhs[p + run] == e) ++run;
  const bool bad_e = e < 0 || e >= a.E;
  const size_t ee = bad_e ? 0 : (size_t)e;
  const uint32_t wbytes = (uint32_t)a.N * (uint32_t)(a.K / 2);
  const uint32_t sbytes = (uint32_t)a.N * (uint32_t)(a.K / GS) * 2u;
  typename S::Ctx cx;
  cx.x = buffer_rsrc(a.x, (uint32_t)a.x_rows * (uint32_t)a.K * 2u);
  cx.w = buffer_rsrc(a.w[0] + ee * (wbytes / 4), wbytes);
  cx.s = buffer_rsrc(a.s[0] + ee * (sbytes / 2), sbytes);
  cx.b = buffer_rsrc(a.b[0] + ee * (sbytes / 2), sbytes);
  cx.w2 = buffer_rsrc(a.w[1] + ee * (wbytes / 4), wbytes);
  cx.s2 = buffer_rsrc(a.s[1] + ee * (sbytes / 2), sbytes);
  cx.b2 = buffer_rsrc(a.b[1] + ee * (sbytes / 2), sbytes);
  cx.split = GLU ? OUTC : S::NB;
  cx.xrows = s_rows;
  cx.xbase = 0;
  cx.K = a.K;
  cx.N = a.N;
  cx.groups = a.K / GS;
  cx.n0 = blockIdx.x * OUTC;
  cx.lane = tid & 63;
  cx.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  cx.sb_base = 0;
  float* red = reinterpret_cast<float*>(dfmi_smem);
  for (int g0 = 0; g0 < run; g0 += 16) {
    const int rows = min(16, run - g0);
    if (g0 > 0 && tid < 16) {  // later row blocks of a long run
      const int pp = p + g0 + min(tid, rows - 1);
      s_lhs[tid] = a.lhs ? a.lhs[pp] : pp;
    }
    __syncthreads();
    if (tid < 16) {
      // rows past the run repeat its last pair; invalid ids read row 0 and
      // are reported as NaN below
      int xr = s_lhs[min(tid, rows - 1)];
      if (xr < 0 || xr >= a.x_rows) xr = 0;
      s_rows[tid] = xr;
    }
    __syncthreads();
    cx.M = rows;
    f32x4 acc[S::NT][1];
#pragma unroll
    for (int t = 0; t < S::NT; ++t) acc[t][0] = zero4();
    if (!bad_e) S::run(cx, 0, a.K / S::CK, acc);
    // sum the 4 wavefronts' partial tiles through LDS (every DMA has landed)
    __syncthreads();
    {
      float* mine = red + cx.wave * S::RED_FLOATS;
#pragma unroll
      for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) mine[(t * 4 + j) * 64 + cx.lane] = acc[t][0][j];
    }
    __syncthreads();
    constexpr int OUT = OUTC * 16;  // output elements: tiles 0 .. OUTC/16-1
    for (int el = tid; el < OUT; el += 256) {
      float v = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        v += red[w * S::RED_FLOATS + el];
        if (GLU) u += red[w * S::RED_FLOATS + OUT + el];  // up tile t + OUTC/16
      }
      const int l = el & 63, j = (el >> 6) & 3, t = el >> 8;
      const int m = 4 * (l >> 4) + j;
      const int n = cx.n0 + t * 16 + (l & 15);
      if (m < rows && n < a.N) {
        const int pp = p + g0 + m;
        const int xrow = s_lhs[m];
        float out;
        if (bad_e || xrow < 0 || xrow >= a.x_rows) {
          out = __builtin_nanf("");
        } else if (GLU) {
          out = silu_mul<Tag>(rnd<Tag>(v), rnd<Tag>(u));
        } else {
          out = v;
        }
        a.y[(int64_t)pp * a.N + n] = Num<Tag>::f2h(out);
      }
    }
    __syncthreads();  // s_lhs, s_rows and the LDS stages are reused by the next row block
  }
}

// ---------------------------------------------------------------------------
// Persistent gather (K % 512 == 0, K / GS <= 32, P <= kPersistMaxPairs).  One
// workgroup of 8 wavefronts per CU runs the streaming main loop (Stream<...,
// 8 wavefronts, 4-piece scale windows>) over a sequence of work units; a unit
// is (segment, block of OUTC output columns), a segment being consecutive
// pairs of one expert, cut every 16 pairs.  The pipeline (three stages in
// flight) runs across unit boundaries: a unit's first stages and its scale
// window are fetched while the previous unit computes, instead of every
// workgroup paying its own pipeline fill (measured: about 5 µs of a 14 µs
// workgroup of the per-run kernel).  Units are dealt round-robin; they cost
// the same (every unit streams 64 weight rows over the whole K).  Every
// workgroup builds the segment table from the pair ids itself (one pass over
// at most 8 KB).
//
// Waits count this wavefront's loads exactly: every wavefront issues the
// same DMA instructions per chunk (CHUNK_DMA) and per scale window (SB_DMA),
// so the number of loads issued after any chunk is known.  The epilogue's
// output stores are left out of the count: loads complete in order among
// themselves, but a store may complete before an older load, so a pending
// store can only make a wait longer, never let it pass early.
constexpr int kPersistMaxPairs = 1024;
constexpr int kPersistGroups = 256;  // workgroups: one per CU
constexpr int kPersistSbBufs = 4;    // scale windows in flight: units in flight <= 4
constexpr int kPersistStages = 3;

template <typename Tag, int GS>
struct PersistLayout {
  using S = Stream<Tag, GS, 1, 8, 4>;
  static_assert(S::DEPTH == kPersistStages, "stages");
  // [0, S::LDS_BYTES): the stream's window 0 and stages; then windows 1..3,
  // the run-start and segment-start masks, the pair tables and the segment
  // starts
  static constexpr int SB_EXTRA = S::LDS_BYTES;
  static constexpr int RUNMASK = SB_EXTRA + (kPersistSbBufs - 1) * S::SBBUF;  // u64[P / 64]
  static constexpr int SEGMASK = RUNMASK + 8 * (kPersistMaxPairs / 64);       // u64[P / 64]
  static constexpr int RHS = SEGMASK + 8 * (kPersistMaxPairs / 64);            // int[P]
  static constexpr int LHS = RHS + 4 * kPersistMaxPairs;   // int[P]: raw activation rows
  static constexpr int XR = LHS + 4 * kPersistMaxPairs;    // int[P]: rows clamped to valid
  static constexpr int SEG = XR + 4 * kPersistMaxPairs;    // int[P + 1]: segment starts, P
  static constexpr int NSEG = SEG + 4 * (kPersistMaxPairs + 1);
  static constexpr int BYTES = NSEG + 16;
  static_assert(BYTES <= 160 * 1024, "LDS");
  static_assert(S::XBUF == 4 * S::RED_FLOATS * 4 && S::WBUF == 4 * S::RED_FLOATS * 4,
                "epilogue: four wavefronts' partial tiles per activation or weight stage");
  __device__ static inline uint32_t sb_base(int unit) {
    const int k = unit & (kPersistSbBufs - 1);
    return k == 0 ? 0u : (uint32_t)(SB_EXTRA + (k - 1) * S::SBBUF);
  }
};

template <typename Tag, int GS, bool GLU>
__global__ __launch_bounds__(512) void gather_persist_kernel(GatherArgs a) {
  using LY = PersistLayout<Tag, GS>;
  using S = typename LY::S;
  constexpr int OUTC = GLU ? S::NB / 2 : S::NB;  // output columns per unit
  constexpr int OUT = OUTC * 16;                 // output elements of a 16-row block
  constexpr int PER = OUT / 512;                 // per thread
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint64_t* t_run = reinterpret_cast<uint64_t*>(dfmi_smem + LY::RUNMASK);
  uint64_t* t_segm = reinterpret_cast<uint64_t*>(dfmi_smem + LY::SEGMASK);
  int* t_rhs = reinterpret_cast<int*>(dfmi_smem + LY::RHS);
  int* t_lhs = reinterpret_cast<int*>(dfmi_smem + LY::LHS);
  int* t_xr = reinterpret_cast<int*>(dfmi_smem + LY::XR);
  int* t_seg = reinterpret_cast<int*>(dfmi_smem + LY::SEG);
  int* t_nseg = reinterpret_cast<int*>(dfmi_smem + LY::NSEG);
  const int P = a.P;
  // the arguments as plain values (lambdas below capture these, never the
  // argument struct itself, whose address would put it in scratch memory)
  const uint16_t* const ax = a.x;
  const int64_t x_rows = a.x_rows;
  const uint32_t* const aw0 = a.w[0];
  const uint32_t* const aw1 = a.w[1];
  const uint16_t* const as0 = a.s[0];
  const uint16_t* const as1 = a.s[1];
  const uint16_t* const ab0 = a.b[0];
  const uint16_t* const ab1 = a.b[1];
  const int32_t* const alhs = a.lhs;
  const int32_t* const arhs = a.rhs;
  uint16_t* const ay = a.y;
  const int K = a.K, N = a.N, E = a.E;

  // --- segment table: pairs -> runs of one expert -> segments of <= 16 pairs
  for (int i = tid; i < P; i += 512) {
    const int l = alhs ? alhs[i] : i;
    t_rhs[i] = arhs[i];
    t_lhs[i] = l;
    t_xr[i] = (l < 0 || l >= x_rows) ? 0 : l;  // invalid rows read row 0, reported as NaN
  }
  __syncthreads();
  const int nw = (P + 63) / 64;
  for (int i = wave; i < nw; i += 8) {  // run starts
    const int p = 64 * i + lane;
    const bool st = p < P && (p == 0 || t_rhs[p] != t_rhs[p - 1]);
    const uint64_t m = __ballot(st);
    if (lane == 0) t_run[i] = m;
  }
  __syncthreads();
  for (int i = wave; i < nw; i += 8) {  // segment starts: run starts and every 16th pair of a run
    const int p = 64 * i + lane;
    bool sg = false;
    if (p < P) {
      int w = i;
      uint64_t m = t_run[w] & (lane == 63 ? ~0ull : ((2ull << lane) - 1ull));
      while (m == 0) m = t_run[--w];  // ends: pair 0 starts a run
      const int rs = 64 * w + 63 - __clzll((long long)m);
      sg = ((p - rs) & 15) == 0;
    }
    const uint64_t m2 = __ballot(sg);
    if (lane == 0) t_segm[i] = m2;
  }
  __syncthreads();
  if (wave == 0) {  // compact the segment starts in order
    int base = 0;
    for (int i = 0; i < nw; ++i) {
      const uint64_t m = t_segm[i];
      if ((m >> lane) & 1ull) t_seg[base + __popcll(m & ((1ull << lane) - 1ull))] = 64 * i + lane;
      base += __popcll(m);
    }
    if (lane == 0) {
      t_seg[base] = P;
      *t_nseg = base;
    }
  }
  __syncthreads();
  const int nseg = __builtin_amdgcn_readfirstlane(*t_nseg);
  const int ncb = (N + OUTC - 1) / OUTC;
  const int units = nseg * ncb;
  const int bid = blockIdx.x, G = gridDim.x;
  const int n_local = bid < units ? (units - bid + G - 1) / G : 0;
  const int C = K / S::CK;  // chunks per unit
  const int V = n_local * C;  // this workgroup's chunks
  if (V == 0) return;         // uniform

  // --- the streaming pipeline over this workgroup's units
  const uint32_t wbytes = (uint32_t)N * (uint32_t)(K / 2);
  const uint32_t sbytes = (uint32_t)N * (uint32_t)(K / GS) * 2u;
  const int npieces = (K / GS + 7) / 8;
  constexpr int SPLIT = GLU ? OUTC : S::NB;  // rows >= SPLIT: the up weight set
  static_assert(S::SB_DMA == 1 && S::NB / S::SB_RPI == 4, "one window instruction per wavefront");
  // the unit being issued, as plain values carried across the loop (buffer
  // resources are rebuilt at each use: a runtime choice between resources
  // is compiled into a table in scratch memory, a choice between base
  // pointers is not)
  const uint32_t* iw0 = aw0;
  const uint32_t* iw1 = aw1;
  const uint16_t* is0 = as0;
  const uint16_t* is1 = as1;
  const uint16_t* ib0 = ab0;
  const uint16_t* ib1 = ab1;
  int ip0 = 0, irows = 1, in0 = 0, iunit = 0;
  typename S::Lane L;
  int ops = 0;  // loads (DMA instructions) this wavefront has issued
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(ax, (uint32_t)x_rows * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(ay, (uint32_t)((int64_t)P * N * 2));
  const DqConst dq = dq_const<Tag>();
  f32x4 acc[S::NT][1];

  // Issue chunk vi: a unit's first chunk is preceded by its scale window.
  auto issue = [&](int vi) __attribute__((always_inline)) {
    const int j = __builtin_amdgcn_readfirstlane(vi / C);
    const int c = __builtin_amdgcn_readfirstlane(vi - j * C);
    const int stage = __builtin_amdgcn_readfirstlane(vi % kPersistStages);
    typename S::Ctx cx;  // what lane_setup and issue_x read
    cx.x = xr;
    cx.split = SPLIT;
    cx.xbase = 0;
    cx.K = K;
    cx.N = N;
    cx.groups = K / GS;
    cx.lane = lane;
    cx.wave = wave;
    if (c == 0) {  // a new unit: its weights, rows and scale window
      const int u = bid + j * G;
      const int sidx = u / ncb;
      const int cb = u - sidx * ncb;
      ip0 = __builtin_amdgcn_readfirstlane(t_seg[sidx]);
      irows = __builtin_amdgcn_readfirstlane(t_seg[sidx + 1]) - ip0;
      const int e = __builtin_amdgcn_readfirstlane(t_rhs[ip0]);
      const size_t ee = (e < 0 || e >= E) ? 0 : (size_t)e;
      iw0 = aw0 + ee * (wbytes / 4);
      iw1 = aw1 + ee * (wbytes / 4);
      is0 = as0 + ee * (sbytes / 2);
      is1 = as1 + ee * (sbytes / 2);
      ib0 = ab0 + ee * (sbytes / 2);
      ib1 = ab1 + ee * (sbytes / 2);
      in0 = cb * OUTC;
      iunit = j;
      cx.xrows = t_xr + ip0;
      cx.M = irows;
      cx.n0 = in0;
      L = S::lane_setup(cx);
      // scale / bias window (Stream::issue_sb's layout): one instruction per
      // wavefront, array wave / 4, rows (wave % 4) * SB_RPI ..
      const int arr = wave >> 2;
      const int r0 = (wave & 3) * S::SB_RPI;
      const int r = r0 + lane / S::SBPC_N;
      const int q = (lane % S::SBPC_N) ^ (r % S::SBPC_N);
      const bool second = r0 >= SPLIT;  // wave-uniform
      const int n = in0 + (second ? r - SPLIT : r);
      const uint32_t off = (q < npieces && n < N)
                               ? ((uint32_t)n * (uint32_t)(K / GS) + (uint32_t)q * 8u) * 2u
                               : kNoRow;
      const uint16_t* base = arr ? (second ? ib1 : ib0) : (second ? is1 : is0);
      dma16<kCpolStream>(buffer_rsrc(base, sbytes), off, 0u,
            dfmi_smem + S::SB_OFF + LY::sb_base(iunit) + arr * S::NB * S::SBP + r0 * S::SBP);
      ops += S::SB_DMA;
    }
    cx.xrows = t_xr + ip0;
    cx.M = irows;
    cx.n0 = in0;
    S::issue_x(cx, L, c, stage);
    // weight stage (Stream::issue_w's layout), gate or up set by base pointer
    constexpr int RPI = 64 / S::WPPR;
    const uint32_t uoff = (uint32_t)c * (uint32_t)S::WROW;
#pragma unroll
    for (int i = 0; i < S::W_DMA; ++i) {
      const int r0 = (wave * S::W_DMA + i) * RPI;  // wave-uniform
      const uint32_t* base = r0 >= SPLIT ? iw1 : iw0;
      dma16<kCpolStream>(buffer_rsrc(base, wbytes), L.wg[i], uoff,
            dfmi_smem + S::W_OFF + stage * S::WBUF + r0 * S::WROW);
    }
    ops += S::CHUNK_DMA;
  };
  // Wait until chunk v has landed: the loads issued after it are its
  // successors' chunks and the scale windows of units begun after it (a
  // unit's window precedes its first chunk).
  auto wait_chunk = [&](int v) __attribute__((always_inline)) {
    const int upto = (v + 1) * S::CHUNK_DMA + (v / C + 1) * S::SB_DMA;  // loads up to chunk v
    stage_barrier_n(ops - upto);
  };
  auto read = [&](int v, typename S::Frag& f) __attribute__((always_inline)) {
    typename S::Ctx cr;  // what the fragment reads use: the wave and the unit's window
    cr.wave = wave;
    cr.sb_base = __builtin_amdgcn_readfirstlane(LY::sb_base(v / C));
    S::read_frag(cr, L, __builtin_amdgcn_readfirstlane(v % C),
                 __builtin_amdgcn_readfirstlane(v % kPersistStages), 0, f);
  };
  // Unit j's outputs.  The stage of the chunk after its last one holds the
  // wavefronts' partial tiles: that chunk's fragments are in registers and
  // its next DMA comes after the next wait's barrier.
  auto epilogue = [&](int j, int slot) __attribute__((always_inline)) {
    const int u = bid + j * G;
    const int sidx = u / ncb;
    const int cb = u - sidx * ncb;
    const int p0 = __builtin_amdgcn_readfirstlane(t_seg[sidx]);
    const int rows = __builtin_amdgcn_readfirstlane(t_seg[sidx + 1]) - p0;
    const int e = __builtin_amdgcn_readfirstlane(t_rhs[p0]);
    const bool bad_e = e < 0 || e >= E;
    const int n0 = cb * OUTC;
    float* rx = reinterpret_cast<float*>(dfmi_smem + S::X_OFF + slot * S::XBUF);
    float* rw = reinterpret_cast<float*>(dfmi_smem + S::W_OFF + slot * S::WBUF);
    stage_barrier<15>();  // every wavefront's fragment reads of that stage have returned
    {
      float* mine = (wave < 4 ? rx : rw) + (wave & 3) * S::RED_FLOATS;
#pragma unroll
      for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mine[(t * 4 + r) * 64 + lane] = acc[t][0][r];
    }
    stage_barrier<15>();
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int el = q * 512 + tid;
      float v = 0.f, uu = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const float* src = (w < 4 ? rx : rw) + (w & 3) * S::RED_FLOATS;
        v += src[el];
        if (GLU) uu += src[OUT + el];  // up tile t + OUTC / 16
      }
      const int l = el & 63, jj = (el >> 6) & 3, t = el >> 8;
      const int m = 4 * (l >> 4) + jj;
      const int n = n0 + 16 * t + (l & 15);
      const int xrow = t_lhs[p0 + min(m, rows - 1)];
      float out;
      if (bad_e || xrow < 0 || xrow >= x_rows) {
        out = __builtin_nanf("");
      } else if (GLU) {
        out = silu_mul<Tag>(rnd<Tag>(v), rnd<Tag>(uu));
      } else {
        out = v;
      }
      const uint32_t off =
          (m < rows && n < N) ? (uint32_t)(((int64_t)(p0 + m) * N + n) * 2) : kNoRow;
      __builtin_amdgcn_raw_buffer_store_b16(Num<Tag>::f2h(out), yr, off, 0, 0);
    }
  };

  for (int k = 0; k < kPersistStages && k < V; ++k) issue(k);
  wait_chunk(0);
  typename S::Frag fa, fb;
  read(0, fa);
  // iteration v: chunk v + 1 must be in LDS (v + 2, v + 3 may be in flight);
  // chunk v's fragments are in CUR
#define DFMI_PERSIST_STEP(v, CUR, NXT)                                        \
  do {                                                                        \
    if ((v) + 1 < V) {                                                        \
      wait_chunk((v) + 1);                                                    \
      if ((v) + kPersistStages < V) issue((v) + kPersistStages);              \
      read((v) + 1, NXT);                                                     \
    }                                                                         \
    if ((v) % C == 0) {                                                       \
      _Pragma("unroll") for (int t = 0; t < S::NT; ++t) acc[t][0] = zero4(); \
    }                                                                         \
    S::compute(L, CUR, acc, dq);                                              \
    if ((v) % C == C - 1) epilogue((v) / C, ((v) + 1) % kPersistStages);      \
  } while (0)
  int v = 0;
  for (; v + 1 < V; v += 2) {
    DFMI_PERSIST_STEP(v, fa, fb);
    DFMI_PERSIST_STEP(v + 1, fb, fa);
  }
  if (v < V) DFMI_PERSIST_STEP(v, fa, fb);
#undef DFMI_PERSIST_STEP
}

// ---------------------------------------------------------------------------
// Pair-streaming persistent gather (moe_stream_kernel): K % 256 == 0, gs 64 /
// 128, P <= kMoeMaxPairs, N a multiple of the unit's output columns, and a
// (scale, bias) pair table per expert (dfmi_moe_pairs).  Two workgroups of 8
// wavefronts per CU (80 KB of LDS each) run the 128-row pair-streaming main
// loop (Stream<..., RW = 2, TSB>: two row groups of 4 wavefronts, each
// wavefront a 64-k slice of every 256-k step) over a sequence of work units;
// a unit is (segment, block of 128 weight rows), a segment being consecutive
// pairs of one expert, cut every 16 pairs.  As in gather_persist_kernel the
// pipeline (three stages in flight) runs across unit boundaries, and the
// segment table is built by every workgroup from the pair ids.
//
// Rows of a unit: the matmul's rows n0 .. n0 + 127 of the expert, or for the
// fused SwiGLU 64 output columns n0 .. n0 + 63 laid out per row group rg as
// 32 gate rows (tiles 0, 1) then the same 32 up rows (tiles 2, 3), columns
// n0 + 32 rg ..; the SwiGLU table interleaves the two pair tables the same
// way ([E][K/gs][2N], 32 gate columns then 32 up columns per 64), so a
// block's pairs are 128 consecutive table columns.
//
// Epilogue without a reduction pass: tile T of a row group is finished by
// one of its wavefronts (wavefront T, or T % 2 for the SwiGLU so that gate
// and up meet in one lane); the other three wavefronts leave their partial
// tile in the stage freed by the fragment reads (24 KB), and the finishing
// wavefront adds them to its own in a fixed order and stores.
//
// Units are dealt CU-major: with G = 2H workgroups, workgroup b takes units
// (b % H) + H (2 i + b / H), so the two workgroups that share a CU under the
// dispatcher's round-robin placement split one run of consecutive units.
constexpr int kMoeMaxPairs = 256;
constexpr int kMoeGroups = 512;  // two workgroups per CU
// workspace of the tail split: counters of at most 255 tail units (4 KB),
// then at most 256 pieces x 2 row groups x 4 tiles x 4 x 64 fp32 partials
constexpr size_t kMoeWsCounterBytes = 4096;
constexpr size_t kMoeWsBytes = kMoeWsCounterBytes + (size_t)(kMoeGroups / 2) * 2 * 1024 * 4;

template <typename Tag, int GS>
struct MoeLayout {
  using S = Stream<Tag, GS, 1, 8, 4, 4, 2, true>;
  static_assert(S::DEPTH == kPersistStages && S::NB == 128 && S::CK == 256, "geometry");
  static_assert(S::X_DMA == 1 && S::W_DMA == 2 && S::T_DMA == 1, "DMA counts");
  static_assert(S::XBUF == 8 * 1024 && S::WBUF == 16 * 1024, "partial tiles: 8 + 16 slots");
  static constexpr int RUNM = S::LDS_BYTES;                  // u64[P / 64]: run starts
  static constexpr int SEGM = RUNM + 8 * (kMoeMaxPairs / 64);  // u64[P / 64]: segment starts
  static constexpr int XR = SEGM + 8 * (kMoeMaxPairs / 64);    // u16[P]: row, | 0x8000 invalid
  static constexpr int SEGS = XR + 2 * kMoeMaxPairs;           // u16[P + 1]: segment starts
  static constexpr int SEGE = SEGS + 2 * (kMoeMaxPairs + 2);   // u16[P]: segment expert
  static constexpr int NSEG = SEGE + 2 * kMoeMaxPairs;
  static constexpr int FLAG = NSEG + 4;  // int: this workgroup's piece completed its unit
  static constexpr int BYTES = FLAG + 4;
  static_assert(BYTES <= 80 * 1024, "two workgroups per CU");
  static_assert(RUNM % 8 == 0 && NSEG % 4 == 0, "alignment");
};

// Scalar arguments, what the start needs first: the hardware preloads the
// first 14 dwords into SGPRs (the pair ids, x, the weights, the pair table,
// P, K), so a workgroup reads its pair ids without a scalar-load round trip
// before them; the rest comes from the kernel arguments when first used.
template <typename Tag, int GS, bool GLU>
__global__ __launch_bounds__(512) void moe_stream_kernel(
    const int32_t* g_lhs, const int32_t* g_rhs, const uint16_t* g_x, const uint32_t* g_w0,
    const uint32_t* g_w1, const uint32_t* g_t, int g_P, int g_K, int g_N, int g_E,
    int64_t g_x_rows, uint16_t* g_y, uint32_t* g_wsc, float* g_wsp) {
  GatherArgs a;
  a.x = g_x;
  a.x_rows = g_x_rows;
  a.w[0] = g_w0;
  a.w[1] = g_w1;
  a.s[0] = a.s[1] = nullptr;
  a.b[0] = a.b[1] = nullptr;
  a.lhs = g_lhs;
  a.rhs = g_rhs;
  a.t = g_t;
  a.ws_counters = g_wsc;
  a.ws_partials = g_wsp;
  a.y = g_y;
  a.P = g_P;
  a.K = g_K;
  a.N = g_N;
  a.E = g_E;
  a.chunks = 0;
  using LY = MoeLayout<Tag, GS>;
  using S = typename LY::S;
  constexpr int OUTC = GLU ? 64 : 128;  // output columns per unit
  constexpr int C_STEP_X = S::CK * 2;   // activation bytes per row and step
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave & 3, rg = wave >> 2;
  uint64_t* t_run = reinterpret_cast<uint64_t*>(dfmi_smem + LY::RUNM);
  uint64_t* t_segm = reinterpret_cast<uint64_t*>(dfmi_smem + LY::SEGM);
  uint16_t* t_xr = reinterpret_cast<uint16_t*>(dfmi_smem + LY::XR);
  uint16_t* t_seg = reinterpret_cast<uint16_t*>(dfmi_smem + LY::SEGS);
  uint16_t* t_se = reinterpret_cast<uint16_t*>(dfmi_smem + LY::SEGE);
  int* t_nseg = reinterpret_cast<int*>(dfmi_smem + LY::NSEG);
  int* t_flag = reinterpret_cast<int*>(dfmi_smem + LY::FLAG);
  const int P = a.P;
  // the arguments as plain values (see gather_persist_kernel)
  const uint16_t* const ax = a.x;
  const int64_t x_rows = a.x_rows;
  const uint32_t* const aw0 = a.w[0];
  const uint32_t* const aw1 = a.w[1];
  const uint32_t* const at = a.t;
  const int32_t* const alhs = a.lhs;
  const int32_t* const arhs = a.rhs;
  uint16_t* const ay = a.y;
  uint32_t* const wsc = a.ws_counters;
  float* const wsp = a.ws_partials;
  const int K = a.K, N = a.N, E = a.E;
  const int NTC = GLU ? 2 * N : N;  // pair table columns per group

  // --- segment table (P <= 256: pair p is thread p of wavefronts 0..3)
  int e_p = 0;
  bool st = false;  // pair tid starts a run
  if (tid < P) {
    const int l = alhs ? alhs[tid] : tid;
    t_xr[tid] = (uint16_t)((l < 0 || l >= x_rows) ? 0x8000 : l);
    e_p = arhs[tid];
    st = tid == 0 || e_p != arhs[tid - 1];
  }
  if (wave < 4) {
    const uint64_t m = __ballot(st);
    if (lane == 0) t_run[wave] = m;
  }
  __syncthreads();
  const int nw = (P + 63) / 64;
  if (wave < nw) {  // segment starts: run starts and every 16th pair of a run
    bool sg = false;
    if (tid < P) {
      int w = wave;
      uint64_t m = t_run[w] & (lane == 63 ? ~0ull : ((2ull << lane) - 1ull));
      while (m == 0) m = t_run[--w];  // ends: pair 0 starts a run
      const int rs = 64 * w + 63 - __clzll((long long)m);
      sg = ((tid - rs) & 15) == 0;
    }
    const uint64_t m2 = __ballot(sg);
    if (lane == 0) t_segm[wave] = m2;
  }
  __syncthreads();
  if (wave < nw) {  // compaction: each wavefront places its own segment starts
    int base = 0;
    for (int i = 0; i < wave; ++i) base += __popcll(t_segm[i]);
    const uint64_t m = t_segm[wave];
    if ((m >> lane) & 1ull) {
      const int s = base + __popcll(m & ((1ull << lane) - 1ull));
      t_seg[s] = (uint16_t)tid;
      t_se[s] = (uint16_t)((e_p < 0 || e_p >= E) ? 0xFFFF : e_p);
    }
    if (wave == nw - 1 && lane == 0) {
      const int total = base + __popcll(m);
      t_seg[total] = (uint16_t)P;
      *t_nseg = total;
    }
  }
  __syncthreads();
  const int nseg = __builtin_amdgcn_readfirstlane(*t_nseg);
  const int ncb = N / OUTC;
  const int units = nseg * ncb;
  const int bid = blockIdx.x, G = gridDim.x;
  const int H = G / 2, h = bid % H, sh = bid / H;  // CU h, slot sh
  const int C = K / S::CK;  // steps per unit
  // Tail split: with R whole rounds of H units, the r units of the last round
  // are cut along K into SP pieces of PC = C / SP steps, one piece per CU, so
  // every CU streams R units plus at most one piece; the pieces' partial
  // tiles meet in the workspace and the last one to arrive finishes the unit.
  // Only with a workspace; pieces of >= 2 steps where units have >= 4 (1-step
  // pieces there cost more in exchanges than they save), of 1 step for
  // 2-step units (measured on the 40-layer sweep: SwiGLU units of 8 steps,
  // down units of 2).
  const int R = units / H, r = units - R * H;
  int SP = 1;
  if (wsc && r > 0 && C >= 2) {
    SP = min(H / r, C >= 4 ? C / 2 : C);
    while (SP > 1 && C % SP) --SP;
  }
  SP = __builtin_amdgcn_readfirstlane(SP);
  const int whole = SP > 1 ? R * H : units;
  // whole units of this workgroup: h + H q with q = sh, sh + 2, ...
  const int qmax = whole > h ? (whole - h + H - 1) / H : 0;
  const int n_whole = qmax > sh ? (qmax - sh + 1) / 2 : 0;
  // its piece (CU h < r SP): taken by the slot with fewer whole units
  const bool has_piece = SP > 1 && h < r * SP && sh == (R & 1);
  const int PC = C / SP;
  // The piece's steps come first, then the whole units': its exchange then
  // overlaps the CU's streaming instead of ending the launch (the lighter
  // slot's stall there lets the other slot stream faster).
  const int PF = has_piece ? PC : 0;     // steps of the piece
  const int V = PF + n_whole * C;        // this workgroup's steps
  if (V == 0) return;                    // uniform
  const int tu = h / SP, ppart = h - tu * SP;  // the piece: tail unit, part
  // Positions carried across the loop (uniform, no divisions per step): the
  // issue side runs the pipeline depth ahead of the compute side.
  int is_next = 0, is_c = 0, is_q = 0;    // issue: next unit start, k step, whole units begun
  int cs_next = 0;                        // compute: next unit start
  int ce_next = PF > 0 ? PF - 1 : C - 1;  // compute: next unit end
  int ep_q = 0;                           // epilogue: whole units finished

  const uint32_t wbytes = (uint32_t)N * (uint32_t)(K / 2);
  const uint32_t wwords = wbytes / 4;
  const uint32_t twords = (uint32_t)(K / GS) * (uint32_t)NTC;
  // the unit being issued, as plain values carried across the loop
  const uint32_t* iw0 = aw0;
  const uint32_t* iw1 = aw1;
  const uint32_t* it = at;
  uint32_t lxg = kNoRow, lwg0 = 0, lwg1 = 0, ltg = kNoRow;
  int ops = 0;  // loads (DMA instructions) this wavefront has issued
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(ax, (uint32_t)x_rows * (uint32_t)K * 2u);
  const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(ay, (uint32_t)((int64_t)P * N * 2));
  const DqConst dq = dq_const<Tag>();
  const u32x4 ones = S::ones_operand();
  // unit-independent fragment offsets
  typename S::Lane L;
  {
    typename S::Ctx cx;
    cx.x = xr;
    cx.w = xr;
    cx.t = xr;
    cx.dense();
    cx.K = K;
    cx.M = 1;
    cx.N = N;
    cx.groups = K / GS;
    cx.n0 = 0;
    cx.lane = lane;
    cx.wave = wave;
    L = S::lane_setup(cx);
  }
  f32x4 acc[S::NT][1];

  // Issue step vi: a unit's first step sets the unit's lane offsets.
  auto issue = [&](int vi) __attribute__((always_inline)) {
    const bool first = vi == is_next;  // a unit's (or the piece's) first step
    if (first) {
      is_c = vi < PF ? ppart * PC : 0;
      is_next = vi < PF ? PF : vi + C;
    }
    const int c = __builtin_amdgcn_readfirstlane(is_c);
    ++is_c;
    const int stage = __builtin_amdgcn_readfirstlane(vi % kPersistStages);
    if (first) {
      const int u = __builtin_amdgcn_readfirstlane(vi < PF ? whole + tu
                                                           : h + H * (2 * is_q++ + sh));
      const int sidx = u / ncb;
      const int cb = u - sidx * ncb;
      const int p0 = __builtin_amdgcn_readfirstlane((int)t_seg[sidx]);
      const int rows = __builtin_amdgcn_readfirstlane((int)t_seg[sidx + 1]) - p0;
      const int e = __builtin_amdgcn_readfirstlane((int)t_se[sidx]);
      const size_t ee = e == 0xFFFF ? 0 : (size_t)e;
      iw0 = aw0 + ee * wwords;
      iw1 = aw1 + ee * wwords;
      it = at + ee * twords;
      const int n0 = cb * OUTC;
      {  // activation rows 2 wave, 2 wave + 1; lane piece (lane % 32) ^ (row & 15)
        const int r = 2 * wave + (lane >> 5);
        const int piece = (lane & 31) ^ (r & 15);
        const int xrow = t_xr[p0 + min(r, rows - 1)] & 0x7fff;
        lxg = r < rows ? (uint32_t)xrow * (uint32_t)K * 2u + (uint32_t)piece * 16u : kNoRow;
      }
      {  // weight rows (2 wave + i) * 8 + lane / 8; piece (lane % 8) ^ (row % 8)
        uint32_t wg[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int R = (2 * wave + i) * 8 + (lane >> 3);
          const int piece = (lane & 7) ^ (R & 7);
          const int n = GLU ? n0 + 32 * (R >> 6) + (R & 31) : n0 + R;
          wg[i] = (uint32_t)n * (uint32_t)(K / 2) + (uint32_t)piece * 16u;
        }
        lwg0 = wg[0];
        lwg1 = wg[1];
      }
      {  // pairs: stage bytes wave TPB + 16 lane = group o / 512, rows (o % 512) / 4 ..
        const int o = wave * S::TPB + 16 * lane;
        const int col = (GLU ? 2 * n0 : n0) + (o % (4 * S::NB)) / 4;
        ltg = lane < S::TLANES
                  ? ((uint32_t)(o / (4 * S::NB)) * (uint32_t)NTC + (uint32_t)col) * 4u
                  : kNoRow;
      }
    }
    dma16(xr, lxg, (uint32_t)c * (uint32_t)C_STEP_X,
          dfmi_smem + S::X_OFF + stage * S::XBUF + wave * 1024);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = (2 * wave + i) * 8;  // wave-uniform
      const uint32_t* base = (GLU && (r0 & 63) >= 32) ? iw1 : iw0;
      dma16<kCpolStream>(buffer_rsrc(base, wbytes), i ? lwg1 : lwg0, (uint32_t)c * (uint32_t)S::WROW,
            dfmi_smem + S::W_OFF + stage * S::WBUF + r0 * S::WROW);
    }
    if (lane < S::TLANES)
      dma16<kCpolStream>(buffer_rsrc(it, twords * 4u), ltg, (uint32_t)c * (uint32_t)(S::GPC * 4 * NTC),
            dfmi_smem + S::T_OFF + stage * S::SBS + wave * S::TPB);
    ops += S::CHUNK_DMA;
  };
  // Wait until step v has landed: the loads issued after it are its
  // successors' (uncounted output stores only lengthen a wait).
  auto wait_chunk = [&](int v) __attribute__((always_inline)) {
    stage_barrier_n(ops - (v + 1) * S::CHUNK_DMA);
  };
  auto read = [&](int v, typename S::Frag& f) __attribute__((always_inline)) {
    typename S::Ctx cr;
    cr.wave = wave;
    cr.sb_base = 0;
    S::read_frag(cr, L, 0, __builtin_amdgcn_readfirstlane(v % kPersistStages), 0, f);
  };
  // Partial tile slot k (0 .. 23) of the free stage: 8 in its activation
  // part, 16 in its weight part.
  auto slot_ptr = [&](int slot, int k) __attribute__((always_inline)) {
    return reinterpret_cast<float*>(
        dfmi_smem + (k < 8 ? S::X_OFF + slot * S::XBUF + k * 1024
                           : S::W_OFF + slot * S::WBUF + (k - 8) * 1024));
  };
  // Outputs of the unit that ends at step v (the stage of the step after it
  // is free: its fragments are in registers and its next DMA follows the
  // next barrier).  A piece instead publishes its partial tiles; the last
  // piece of a unit to arrive sums all of them in part order and finishes
  // (the others return from here and go on to their whole units).
  auto epilogue = [&](int v, int slot) __attribute__((always_inline)) {
    const bool piece = v < PF;  // uniform: the workgroup's first work item
    const int u = __builtin_amdgcn_readfirstlane(piece ? whole + tu : h + H * (2 * ep_q++ + sh));
    const int sidx = u / ncb;
    const int cb = u - sidx * ncb;
    const int p0 = __builtin_amdgcn_readfirstlane((int)t_seg[sidx]);
    const int rows = __builtin_amdgcn_readfirstlane((int)t_seg[sidx + 1]) - p0;
    const bool bad_e = __builtin_amdgcn_readfirstlane((int)t_se[sidx]) == 0xFFFF;
    const int n0 = cb * OUTC;
    stage_barrier<15>();  // every wavefront's fragment reads of that stage have returned
#pragma unroll
    for (int T = 0; T < 4; ++T) {
      const int fin = GLU ? (T & 1) : T;  // the finishing wavefront of tile T
      if (fin != kw) {
        const int k = rg * 12 + T * 3 + (kw < fin ? kw : kw - 1);
        reinterpret_cast<f32x4*>(slot_ptr(slot, k))[lane] = acc[T][0];  // one 16-byte write
      }
    }
    stage_barrier<15>();
    const bool finisher = GLU ? kw < 2 : true;
    // the finished tiles (tile kw, and kw + 2 for the SwiGLU): this
    // wavefront's own partials, selected without indexing registers, plus
    // the other three wavefronts'
    float g[4], up[4];
    if (finisher) {
      f32x4 own0, own1;
      if constexpr (GLU) {
        own0 = kw == 0 ? acc[0][0] : acc[1][0];
        own1 = kw == 0 ? acc[2][0] : acc[3][0];
      } else {
        own0 = kw == 0 ? acc[0][0] : (kw == 1 ? acc[1][0] : (kw == 2 ? acc[2][0] : acc[3][0]));
        own1 = own0;
      }
      const int k0 = rg * 12 + kw * 3, k1 = rg * 12 + (kw + 2) * 3;  // their slots
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        g[q] = own0[q];
        up[q] = own1[q];
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) {  // one 16-byte read per partial tile
        const f32x4 a = reinterpret_cast<const f32x4*>(slot_ptr(slot, k0 + i))[lane];
#pragma unroll
        for (int q = 0; q < 4; ++q) g[q] += a[q];
        if (GLU) {
          const f32x4 b = reinterpret_cast<const f32x4*>(slot_ptr(slot, k1 + i))[lane];
#pragma unroll
          for (int q = 0; q < 4; ++q) up[q] += b[q];
        }
      }
    }
    if (piece) {
      // partial tiles of part ppart: [tail unit][part][row group][tile][reg][lane]
      float* mine = wsp + ((size_t)(tu * SP + ppart) * 2 + rg) * 1024;
      if (finisher) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __hip_atomic_store(mine + (kw * 4 + q) * 64 + lane, g[q], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          if (GLU)
            __hip_atomic_store(mine + ((kw + 2) * 4 + q) * 64 + lane, up[q], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      // every partial store of the workgroup has completed (and the next
      // steps' DMAs in flight have landed: stores and loads share vmcnt)
      stage_barrier<0>();
      if (tid == 0) {
        const unsigned prev =
            __hip_atomic_fetch_add(&wsc[tu], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *t_flag = prev == (unsigned)(SP - 1) ? 1 : 0;
      }
      stage_barrier<0>();
      if (!__builtin_amdgcn_readfirstlane(*t_flag)) return;
      if (finisher) {
        const float* first = wsp + ((size_t)tu * SP * 2 + rg) * 1024;
#pragma unroll
        for (int q = 0; q < 4; ++q) g[q] = up[q] = 0.f;
        for (int p = 0; p < SP; ++p) {  // part order: independent of arrival order
          const float* pp = first + (size_t)p * 2 * 1024;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            g[q] += __hip_atomic_load(pp + (kw * 4 + q) * 64 + lane, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            if (GLU)
              up[q] += __hip_atomic_load(pp + ((kw + 2) * 4 + q) * 64 + lane, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      if (tid == 0) __hip_atomic_exchange(&wsc[tu], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (finisher) {
      const int col = lane & 15, kg = lane >> 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q >= rows) break;  // uniform: no lane of the wavefront holds an output row
        const int m = 4 * kg + q;
        const int n = GLU ? n0 + 32 * rg + 16 * kw + col : n0 + 64 * rg + 16 * kw + col;
        const int xrow = t_xr[p0 + min(m, rows - 1)];
        float out;
        if (bad_e || (xrow & 0x8000)) {
          out = __builtin_nanf("");
        } else if (GLU) {
          out = silu_mul<Tag>(rnd<Tag>(g[q]), rnd<Tag>(up[q]));
        } else {
          out = g[q];
        }
        const uint32_t off =
            m < rows ? (uint32_t)(((int64_t)(p0 + m) * N + n) * 2) : kNoRow;
        __builtin_amdgcn_raw_buffer_store_b16(Num<Tag>::f2h(out), yr, off, 0, 0);
      }
    }
  };

  for (int k = 0; k < kPersistStages && k < V; ++k) issue(k);
  wait_chunk(0);
  typename S::Frag fa, fb;
  read(0, fa);
#define DFMI_MOE_STEP(v, CUR, NXT)                                            \
  do {                                                                        \
    if ((v) + 1 < V) {                                                        \
      wait_chunk((v) + 1);                                                    \
      if ((v) + kPersistStages < V) issue((v) + kPersistStages);              \
      read((v) + 1, NXT);                                                     \
    }                                                                         \
    if ((v) == cs_next) {                                                     \
      _Pragma("unroll") for (int t = 0; t < S::NT; ++t) acc[t][0] = zero4(); \
      cs_next = (v) < PF ? PF : (v) + C;                                      \
    }                                                                         \
    S::compute(L, CUR, acc, dq, ones);                                        \
    if ((v) == ce_next || (v) == V - 1) {                                     \
      epilogue((v), ((v) + 1) % kPersistStages);                              \
      ce_next += C;                                                           \
    }                                                                         \
  } while (0)
  int v = 0;
  for (; v + 1 < V; v += 2) {
    DFMI_MOE_STEP(v, fa, fb);
    DFMI_MOE_STEP(v + 1, fb, fa);
  }
  if (v < V) DFMI_MOE_STEP(v, fa, fb);
#undef DFMI_MOE_STEP
}

template <typename Tag, int GS, bool GLU>
static void launch_moe_stream_t(const GatherArgs& a, int grid, hipStream_t st) {
  using LY = MoeLayout<Tag, GS>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&moe_stream_kernel<Tag, GS, GLU>),
      hipFuncAttributeMaxDynamicSharedMemorySize, LY::BYTES);
  (void)attr;
  hipLaunchKernelGGL((moe_stream_kernel<Tag, GS, GLU>), dim3(grid), dim3(512), LY::BYTES, st,
                     a.lhs, a.rhs, a.x, a.w[0], a.w[1], a.t, a.P, a.K, a.N, a.E, a.x_rows, a.y,
                     a.ws_counters, a.ws_partials);
}

template <typename Tag, bool GLU>
static void launch_moe_stream(const GatherArgs& a, int gs, int grid, hipStream_t st) {
  if (gs == 64) launch_moe_stream_t<Tag, 64, GLU>(a, grid, st);
  else launch_moe_stream_t<Tag, 128, GLU>(a, grid, st);
}

template <typename Tag, int GS, bool GLU>
static void launch_gather_persist_t(const GatherArgs& a, hipStream_t st) {
  using LY = PersistLayout<Tag, GS>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&gather_persist_kernel<Tag, GS, GLU>),
      hipFuncAttributeMaxDynamicSharedMemorySize, LY::BYTES);
  (void)attr;
  hipLaunchKernelGGL((gather_persist_kernel<Tag, GS, GLU>), dim3(kPersistGroups), dim3(512),
                     LY::BYTES, st, a);
}

template <typename Tag, bool GLU>
static void launch_gather_persist(const GatherArgs& a, int gs, hipStream_t st) {
  if (gs == 32) launch_gather_persist_t<Tag, 32, GLU>(a, st);
  else if (gs == 64) launch_gather_persist_t<Tag, 64, GLU>(a, st);
  else launch_gather_persist_t<Tag, 128, GLU>(a, st);
}

template <typename Tag, int GS, bool GLU, int SBPC>
static void launch_gather_stream_t(const GatherArgs& a, hipStream_t st) {
  using S = Stream<Tag, GS, 1, 4, SBPC>;
  constexpr int OUTC = GLU ? S::NB / 2 : S::NB;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&gather_stream_kernel<Tag, GS, GLU, SBPC>),
      hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS_BYTES);
  (void)attr;
  const dim3 grid((unsigned)((a.N + OUTC - 1) / OUTC), (unsigned)a.P);
  hipLaunchKernelGGL((gather_stream_kernel<Tag, GS, GLU, SBPC>), grid, dim3(256), S::LDS_BYTES,
                     st, a);
}

// The narrow scale window (8 pieces, 64 KB of LDS with 4 wavefronts) keeps
// two workgroups per CU next to the kernel's static index arrays; K ranges
// of more groups take the wide one (80 KB, one workgroup per CU).
template <typename Tag, bool GLU, int GS>
static void launch_gather_stream_gs(const GatherArgs& a, hipStream_t st) {
  if (a.K / GS <= sb_max_groups(8)) launch_gather_stream_t<Tag, GS, GLU, 8>(a, st);
  else launch_gather_stream_t<Tag, GS, GLU, kSbPieces>(a, st);
}

template <typename Tag, bool GLU>
static void launch_gather_stream(const GatherArgs& a, int gs, hipStream_t st) {
  if (gs == 32) launch_gather_stream_gs<Tag, GLU, 32>(a, st);
  else if (gs == 64) launch_gather_stream_gs<Tag, GLU, 64>(a, st);
  else launch_gather_stream_gs<Tag, GLU, 128>(a, st);
}

template <typename Tag, int GS, int NT, bool KFULL, bool GLU>
static void launch_gather_t(const GatherArgs& a, int n_blocks, int waves, hipStream_t st) {
  hipLaunchKernelGGL((gather_kernel<Tag, GS, NT, KFULL, GLU>), dim3(n_blocks, a.P),
                     dim3(64 * waves), 0, st, a);
}

template <typename Tag, int GS, bool GLU>
static void launch_gather_gs(const GatherArgs& a, bool kfull, int nt, int n_blocks, int waves,
                             hipStream_t st) {
  if (nt == 1) {
    if (kfull) launch_gather_t<Tag, GS, 1, true, GLU>(a, n_blocks, waves, st);
    else launch_gather_t<Tag, GS, 1, false, GLU>(a, n_blocks, waves, st);
  } else {
    if (kfull) launch_gather_t<Tag, GS, 2, true, GLU>(a, n_blocks, waves, st);
    else launch_gather_t<Tag, GS, 2, false, GLU>(a, n_blocks, waves, st);
  }
}

template <typename Tag, bool GLU>
static void launch_gather(const GatherArgs& a, int gs, bool kfull, int nt, int n_blocks,
                          int waves, hipStream_t st) {
  if (gs == 32) launch_gather_gs<Tag, 32, GLU>(a, kfull, nt, n_blocks, waves, st);
  else if (gs == 64) launch_gather_gs<Tag, 64, GLU>(a, kfull, nt, n_blocks, waves, st);
  else launch_gather_gs<Tag, 128, GLU>(a, kfull, nt, n_blocks, waves, st);
}

// Shapes moe_stream_kernel takes (with a pair table): 4-bit weights (checked
// by the caller), gs 64 / 128, whole 256-k steps, whole units of 64 (SwiGLU)
// or 128 output columns, at most kMoeMaxPairs pairs, 16-bit row and expert
// ids, 32-bit buffer offsets.
static bool moe_stream_eligible(int64_t x_rows, int64_t P, int64_t K, int64_t N, int64_t E,
                                int gs, bool glu) {
  const int64_t ntc = glu ? 2 * N : N;
  return (gs == 64 || gs == 128) && K >= 256 && K % 256 == 0 && N > 0 &&
         N % (glu ? 64 : 128) == 0 && P >= 1 && P <= kMoeMaxPairs && x_rows <= 32767 &&
         E < 65535 && x_rows * K * 2 < (1ll << 31) && N * (K / 2) < (1ll << 31) &&
         (K / gs) * ntc * 4 < (1ll << 31) && P * N * 2 < (1ll << 31);
}

static int validate_gather(int x_dtype, int64_t x_rows, int64_t P, int64_t K, int64_t N,
                           int64_t E, int gs, int bits) {
  if (x_dtype != DFMI_BF16 && x_dtype != DFMI_F16) {
    set_error("dfmi_gather_qmm: x dtype %d unsupported (bf16 or f16)", x_dtype);
    return DFMI_EINVAL;
  }
  if (bits != 4) {
    set_error("dfmi_gather_qmm: bits=%d unsupported (4)", bits);
    return DFMI_EINVAL;
  }
  if (gs != 32 && gs != 64 && gs != 128) {
    set_error("dfmi_gather_qmm: group_size=%d unsupported (32, 64, 128)", gs);
    return DFMI_EINVAL;
  }
  // no pairs (zero tokens routed) needs no activation rows
  if (P < 0 || N < 0 || E < 1 || x_rows < (P > 0 ? 1 : 0) || K < 32 || K % 32 || K % gs) {
    set_error("dfmi_gather_qmm: bad shape P=%lld K=%lld N=%lld E=%lld x_rows=%lld gs=%d",
              (long long)P, (long long)K, (long long)N, (long long)E, (long long)x_rows, gs);
    return DFMI_EINVAL;
  }
  if (P > 65535 || N >= (1ll << 31) || K >= (1ll << 31) || x_rows >= (1ll << 31) ||
      N * (K / 8) > 0xFFFFFFFFll) {
    set_error("dfmi_gather_qmm: shape too large P=%lld K=%lld N=%lld", (long long)P,
              (long long)K, (long long)N);
    return DFMI_EINVAL;
  }
  return DFMI_OK;
}

static int gather_common(const void* x, int x_dtype, int64_t x_rows, const uint32_t* w0,
                         const void* s0, const void* b0, const uint32_t* w1, const void* s1,
                         const void* b1, const int32_t* lhs_rows, const int32_t* rhs_experts,
                         void* y, int64_t P, int64_t K, int64_t N, int64_t E, int group_size,
                         int bits, bool glu, const uint32_t* pairs, void* workspace,
                         size_t workspace_bytes, void* stream) {
  int rc = validate_gather(x_dtype, x_rows, P, K, N, E, group_size, bits);
  if (rc != DFMI_OK) return rc;
  if (P == 0 || N == 0) return DFMI_OK;
  if (!x || !w0 || !s0 || !b0 || !rhs_experts || !y || (glu && (!w1 || !s1 || !b1))) {
    set_error("dfmi_gather_qmm: null pointer");
    return DFMI_EINVAL;
  }
  if (!aligned16(x) || !aligned16(w0) || !aligned16(s0) || !aligned16(b0) ||
      (glu && (!aligned16(w1) || !aligned16(s1) || !aligned16(b1)))) {
    set_error("dfmi_gather_qmm: x, weights, scales and biases must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  GatherArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.x_rows = x_rows;
  a.w[0] = w0;
  a.s[0] = static_cast<const uint16_t*>(s0);
  a.b[0] = static_cast<const uint16_t*>(b0);
  a.w[1] = glu ? w1 : w0;
  a.s[1] = static_cast<const uint16_t*>(glu ? s1 : s0);
  a.b[1] = static_cast<const uint16_t*>(glu ? b1 : b0);
  a.lhs = lhs_rows;
  a.rhs = rhs_experts;
  a.y = static_cast<uint16_t*>(y);
  a.P = (int)P;
  a.K = (int)K;
  a.N = (int)N;
  a.E = (int)E;
  a.chunks = (int)((K + kChunkK - 1) / kChunkK);
  a.t = pairs;
  const bool ws_ok = workspace && workspace_bytes >= kMoeWsBytes && aligned16(workspace);
  a.ws_counters = ws_ok ? static_cast<uint32_t*>(workspace) : nullptr;
  a.ws_partials =
      ws_ok ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kMoeWsCounterBytes) : nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // pair-streaming persistent loop (a pair table given): whole 256-k steps,
  // 128-row units, two workgroups per CU, the pair ids in 16-bit LDS tables.
  if (pairs && aligned16(pairs) && moe_stream_eligible(x_rows, P, K, N, E, group_size, glu)) {
    const int64_t units_max = P * (N / (glu ? 64 : 128));  // segments <= pairs
    const int grid =
        (int)std::min<int64_t>(kMoeGroups, std::max<int64_t>(2, (units_max + 1) & ~1ll));
    if (glu) {
      if (x_dtype == DFMI_BF16) launch_moe_stream<BF16, true>(a, group_size, grid, st);
      else launch_moe_stream<F16, true>(a, group_size, grid, st);
    } else {
      if (x_dtype == DFMI_BF16) launch_moe_stream<BF16, false>(a, group_size, grid, st);
      else launch_moe_stream<F16, false>(a, group_size, grid, st);
    }
    return check_launch(glu ? "dfmi_gather_qmm_swiglu" : "dfmi_gather_qmm_affine");
  }
  // persistent pipelined loop: whole 512-k steps, a full-K scale window of
  // at most 4 pieces, the pair tables in LDS, 32-bit buffer offsets.
  // Measured on MI355X (16 tokens, top-8 of 256 experts, 40 layers): the
  // SwiGLU pair at K = 2048 56.1 -> 42.2 µs per layer; at K = 512 (one step
  // per unit, an 8-wavefront reduction per step) slower than the general
  // loop (31.1 vs 25.9 µs), so units of one step stay there.
  if (K % 512 == 0 && K >= 1024 && K / group_size <= 32 && P <= kPersistMaxPairs &&
      x_rows * K * 2 < (1ll << 31) && N * (K / 2) < (1ll << 31) && P * N * 2 < (1ll << 31)) {
    if (glu) {
      if (x_dtype == DFMI_BF16) launch_gather_persist<BF16, true>(a, group_size, st);
      else launch_gather_persist<F16, true>(a, group_size, st);
    } else {
      if (x_dtype == DFMI_BF16) launch_gather_persist<BF16, false>(a, group_size, st);
      else launch_gather_persist<F16, false>(a, group_size, st);
    }
    return check_launch(glu ? "dfmi_gather_qmm_swiglu" : "dfmi_gather_qmm_affine");
  }
  // streaming loop: whole 256-k steps, the whole K in one scale / bias
  // window, 32-bit buffer offsets per expert and for the activations.
  // Measured on MI355X (16 tokens, top-8 of 256 experts): equal to the
  // general loop for the SwiGLU pair at K = 2048 and slower for K = 512 (two
  // steps per workgroup do not amortise its pipeline fill), so short K stays
  // on the general loop.
  if (stream_eligible(16, K, N, group_size) && K >= 1024 && x_rows * K * 2 < (1ll << 31) &&
      K / group_size <= sb_max_groups(kSbPieces)) {
    if (glu) {
      if (x_dtype == DFMI_BF16) launch_gather_stream<BF16, true>(a, group_size, st);
      else launch_gather_stream<F16, true>(a, group_size, st);
    } else {
      if (x_dtype == DFMI_BF16) launch_gather_stream<BF16, false>(a, group_size, st);
      else launch_gather_stream<F16, false>(a, group_size, st);
    }
    return check_launch(glu ? "dfmi_gather_qmm_swiglu" : "dfmi_gather_qmm_affine");
  }
  const bool kfull = (K % kChunkK) == 0;
  const int nt = N >= 1024 ? 2 : 1;
  const int n_blocks = (int)((N + 16 * nt - 1) / (16 * nt));
  const int waves = std::max(1, std::min(kMaxWaves, a.chunks));
  if (glu) {
    if (x_dtype == DFMI_BF16) launch_gather<BF16, true>(a, group_size, kfull, nt, n_blocks, waves, st);
    else launch_gather<F16, true>(a, group_size, kfull, nt, n_blocks, waves, st);
  } else {
    if (x_dtype == DFMI_BF16) launch_gather<BF16, false>(a, group_size, kfull, nt, n_blocks, waves, st);
    else launch_gather<F16, false>(a, group_size, kfull, nt, n_blocks, waves, st);
  }
  return check_launch(glu ? "dfmi_gather_qmm_swiglu" : "dfmi_gather_qmm_affine");
}

// out[t, d] = rnd(sum_j scores[t, j] * y[r(t*k + j), d]), fp32, j in order;
// r(p) = y_rows[p] (the pair's row in a sorted y: the unsort mlx-lm's
// SwitchGLU applies before the weighted sum) or p.  A row id outside
// [0, T*k) makes the output NaN.
template <typename Tag>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* y, const int32_t* y_rows,
                                                      const float* scores, uint16_t* out, int T,
                                                      int k, int D) {
  const int t = blockIdx.y;
  const int64_t P = (int64_t)T * k;
  for (int d = blockIdx.x * 256 + threadIdx.x; d < D; d += gridDim.x * 256) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) {
      const int64_t p = (int64_t)t * k + j;
      const int64_t r = y_rows ? (int64_t)y_rows[p] : p;
      const float v = (r >= 0 && r < P) ? Num<Tag>::h2f(y[r * D + d]) : __builtin_nanf("");
      acc = __builtin_fmaf(scores[p], v, acc);
    }
    out[(int64_t)t * D + d] = Num<Tag>::f2h(acc);
  }
}

// The same sums for D % 8 == 0: a lane takes 8 consecutive columns (one
// 16-byte load per pair), one wavefront per 512 columns of a token.  Same fma
// order.  Eight pairs at a time, in two memory round trips: lanes 0..7 load
// the eight pair ids and scores (one vector load each, broadcast with
// readlane), then every lane requests its eight rows before the first fma (an
// out-of-range id loads row 0 and is replaced by NaN after the load).  Lanes
// past D load columns 0..7 and store nothing, so every lane takes part in the
// broadcast.
template <typename Tag>
__global__ __launch_bounds__(64) void combine8_kernel(const uint16_t* y, const int32_t* y_rows,
                                                      const float* scores, uint16_t* out, int T,
                                                      int k, int D) {
  const int t = blockIdx.y;
  const int lane = (int)threadIdx.x;
  const int d0 = (blockIdx.x * 64 + lane) * 8;
  const bool in = d0 < D;
  const int dl = in ? d0 : 0;  // the column this lane loads
  const int64_t P = (int64_t)T * k;
  const int64_t base = (int64_t)t * k;
  const u32x4 nan4 = {0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu};  // NaN in both dtypes
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int j0 = 0; j0 < k; j0 += 8) {
    const int64_t pl = base + min(j0 + (lane & 7), k - 1);  // slots past k: loaded, not used
    const int32_t my_id = y_rows ? y_rows[pl] : (int32_t)pl;
    const float my_sc = scores[pl];
    u32x4 v[8];
    float sc[8];
    bool ok[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = __builtin_amdgcn_readlane(my_id, i);
      sc[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sc), i));
      ok[i] = r >= 0 && r < P;
      v[i] = *reinterpret_cast<const u32x4*>(y + (ok[i] ? r : 0) * D + dl);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // a slot past k leaves acc as it is (a select, no branch)
      const bool use = j0 + i < k;
      const u32x4 w = ok[i] ? v[i] : nan4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __builtin_fmaf(sc[i], Num<Tag>::h2f((uint16_t)(w[e] & 0xFFFFu)), acc[2 * e]);
        const float hi = __builtin_fmaf(sc[i], Num<Tag>::h2f((uint16_t)(w[e] >> 16)), acc[2 * e + 1]);
        acc[2 * e] = use ? lo : acc[2 * e];
        acc[2 * e + 1] = use ? hi : acc[2 * e + 1];
      }
    }
  }
  if (!in) return;
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = (uint32_t)Num<Tag>::f2h(acc[2 * e]) | ((uint32_t)Num<Tag>::f2h(acc[2 * e + 1]) << 16);
  *reinterpret_cast<u32x4*>(out + (int64_t)t * D + d0) = o;
}

}  // namespace dfmi

using namespace dfmi;

extern "C" int dfmi_gather_qmm_affine(const void* x, int x_dtype, int64_t x_rows,
                                      const uint32_t* w_q, const void* scales, const void* biases,
                                      const int32_t* lhs_rows, const int32_t* rhs_experts,
                                      void* y, int64_t P, int64_t K, int64_t N, int64_t E,
                                      int group_size, int bits, void* stream) {
  return gather_common(x, x_dtype, x_rows, w_q, scales, biases, nullptr, nullptr, nullptr,
                       lhs_rows, rhs_experts, y, P, K, N, E, group_size, bits, false, nullptr,
                       nullptr, 0, stream);
}

extern "C" int dfmi_gather_qmm_affine_pairs(const void* x, int x_dtype, int64_t x_rows,
                                            const uint32_t* w_q, const void* scales,
                                            const void* biases, const uint32_t* sb_pairs,
                                            const int32_t* lhs_rows, const int32_t* rhs_experts,
                                            void* y, int64_t P, int64_t K, int64_t N, int64_t E,
                                            int group_size, int bits, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  return gather_common(x, x_dtype, x_rows, w_q, scales, biases, nullptr, nullptr, nullptr,
                       lhs_rows, rhs_experts, y, P, K, N, E, group_size, bits, false, sb_pairs,
                       workspace, workspace_bytes, stream);
}

extern "C" size_t dfmi_gather_workspace_bytes(void) { return kMoeWsBytes; }

extern "C" int dfmi_gather_qmm_swiglu(const void* x, int x_dtype, int64_t x_rows,
                                      const uint32_t* wg_q, const void* g_scales,
                                      const void* g_biases, const uint32_t* wu_q,
                                      const void* u_scales, const void* u_biases,
                                      const int32_t* lhs_rows, const int32_t* rhs_experts,
                                      void* h, int64_t P, int64_t K, int64_t N, int64_t E,
                                      int group_size, int bits, void* stream) {
  return gather_common(x, x_dtype, x_rows, wg_q, g_scales, g_biases, wu_q, u_scales, u_biases,
                       lhs_rows, rhs_experts, h, P, K, N, E, group_size, bits, true, nullptr,
                       nullptr, 0, stream);
}

extern "C" int dfmi_gather_qmm_swiglu_pairs(const void* x, int x_dtype, int64_t x_rows,
                                            const uint32_t* wg_q, const void* g_scales,
                                            const void* g_biases, const uint32_t* wu_q,
                                            const void* u_scales, const void* u_biases,
                                            const uint32_t* sb_pairs, const int32_t* lhs_rows,
                                            const int32_t* rhs_experts, void* h, int64_t P,
                                            int64_t K, int64_t N, int64_t E, int group_size,
                                            int bits, void* workspace, size_t workspace_bytes,
                                            void* stream) {
  return gather_common(x, x_dtype, x_rows, wg_q, g_scales, g_biases, wu_q, u_scales, u_biases,
                       lhs_rows, rhs_experts, h, P, K, N, E, group_size, bits, true, sb_pairs,
                       workspace, workspace_bytes, stream);
}

// Pair tables of expert weights: [E][G][N] from one (scales, biases) set, or
// for the SwiGLU [E][G][2N] interleaving the gate and up sets 32 columns at a
// time (table column 64 (n / 32) + 32 up + n % 32).  Each workgroup
// transposes 64 table columns x 64 groups of one expert through LDS.
__global__ __launch_bounds__(256) void moe_pairs_kernel(const uint16_t* s0, const uint16_t* b0,
                                                        const uint16_t* s1, const uint16_t* b1,
                                                        uint32_t* t, int N, int G) {
  __shared__ uint32_t tile[64][65];
  const bool glu = s1 != nullptr;
  const int ntc = glu ? 2 * N : N;
  const int c0 = blockIdx.x * 64, g0 = blockIdx.y * 64;
  const int64_t e = blockIdx.z;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, gi = i % 64;  // table column c0 + r, group g0 + gi
    const int c = c0 + r, g = g0 + gi;
    uint32_t v = 0;
    if (c < ntc && g < G) {
      const bool up = glu && (c & 32);
      const int n = glu ? 32 * (c >> 6) + (c & 31) : c;
      const int64_t o = (e * N + n) * G + g;
      const uint16_t sv = up ? s1[o] : s0[o];
      const uint16_t bv = up ? b1[o] : b0[o];
      v = (uint32_t)sv | ((uint32_t)bv << 16);
    }
    tile[r][gi] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int gi = i / 64, r = i % 64;
    const int c = c0 + r, g = g0 + gi;
    if (c < ntc && g < G) t[(e * G + g) * ntc + c] = tile[r][gi];
  }
}

extern "C" int dfmi_moe_pairs(const void* scales, const void* biases, const void* up_scales,
                              const void* up_biases, int dtype, int64_t E, int64_t N,
                              int64_t groups, uint32_t* sb_pairs, void* stream) {
  if (dtype != DFMI_BF16 && dtype != DFMI_F16) {
    set_error("dfmi_moe_pairs: dtype %d unsupported (bf16 or f16)", dtype);
    return DFMI_EINVAL;
  }
  const bool glu = up_scales != nullptr || up_biases != nullptr;
  if (E < 0 || N < 0 || groups < 0 || E > 65535 || N >= (1ll << 30) || groups >= (1ll << 30) ||
      (glu && N % 32 != 0) || E * N * groups * (glu ? 2 : 1) >= (1ll << 40)) {
    set_error("dfmi_moe_pairs: bad shape E=%lld N=%lld groups=%lld%s", (long long)E,
              (long long)N, (long long)groups, glu ? " (SwiGLU: N a multiple of 32)" : "");
    return DFMI_EINVAL;
  }
  if (E == 0 || N == 0 || groups == 0) return DFMI_OK;
  if (!scales || !biases || !sb_pairs || (glu && (!up_scales || !up_biases))) {
    set_error("dfmi_moe_pairs: null pointer");
    return DFMI_EINVAL;
  }
  const int64_t ntc = glu ? 2 * N : N;
  const dim3 grid((unsigned)((ntc + 63) / 64), (unsigned)((groups + 63) / 64), (unsigned)E);
  hipLaunchKernelGGL(moe_pairs_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases),
                     static_cast<const uint16_t*>(up_scales),
                     static_cast<const uint16_t*>(up_biases), sb_pairs, (int)N, (int)groups);
  return check_launch("dfmi_moe_pairs");
}

extern "C" int dfmi_moe_combine(const void* y, int y_dtype, const int32_t* y_rows,
                                const float* scores, void* out, int64_t T, int64_t k, int64_t D,
                                void* stream) {
  if (y_dtype != DFMI_BF16 && y_dtype != DFMI_F16) {
    set_error("dfmi_moe_combine: dtype %d unsupported (bf16 or f16)", y_dtype);
    return DFMI_EINVAL;
  }
  if (T < 0 || k < 1 || D < 0 || T > 65535 || T * k * D >= (1ll << 40)) {
    set_error("dfmi_moe_combine: bad shape T=%lld k=%lld D=%lld", (long long)T, (long long)k,
              (long long)D);
    return DFMI_EINVAL;
  }
  if (T == 0 || D == 0) return DFMI_OK;
  if (!y || !scores || !out) {
    set_error("dfmi_moe_combine: null pointer");
    return DFMI_EINVAL;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D % 8 == 0 && aligned16(y) && aligned16(out)) {
    const dim3 grid((unsigned)((D / 8 + 63) / 64), (unsigned)T);
    if (y_dtype == DFMI_BF16)
      hipLaunchKernelGGL(combine8_kernel<BF16>, grid, dim3(64), 0, st,
                         static_cast<const uint16_t*>(y), y_rows, scores,
                         static_cast<uint16_t*>(out), (int)T, (int)k, (int)D);
    else
      hipLaunchKernelGGL(combine8_kernel<F16>, grid, dim3(64), 0, st,
                         static_cast<const uint16_t*>(y), y_rows, scores,
                         static_cast<uint16_t*>(out), (int)T, (int)k, (int)D);
    return check_launch("dfmi_moe_combine");
  }
  const int gx = (int)std::min<int64_t>((D + 255) / 256, 64);
  if (y_dtype == DFMI_BF16)
    hipLaunchKernelGGL(combine_kernel<BF16>, dim3(gx, (unsigned)T), dim3(256), 0, st,
                       static_cast<const uint16_t*>(y), y_rows, scores,
                       static_cast<uint16_t*>(out), (int)T, (int)k, (int)D);
  else
    hipLaunchKernelGGL(combine_kernel<F16>, dim3(gx, (unsigned)T), dim3(256), 0, st,
                       static_cast<const uint16_t*>(y), y_rows, scores,
                       static_cast<uint16_t*>(out), (int)T, (int)k, (int)D);
  return check_launch("dfmi_moe_combine");
}
