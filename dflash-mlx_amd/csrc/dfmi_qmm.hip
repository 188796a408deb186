// Dense affine int4 qmm: y[M,N] = x[M,K] . dequant(W)^T on gfx950.
//
// Grid: one workgroup per 16*NT output columns (and per 32-row block of M
// when M > 32).  The workgroup's W wavefronts split K between them and sum
// their partial tiles through LDS (Core::reduce), so every output element is
// written once, by one workgroup, with no atomics and no device-scope fence.
// NT grows with N (1, 2, 4 tiles per wavefront) so that every workgroup
// streams enough weight bytes to amortise its activation reads (x is read
// from L2 by every workgroup: x bytes / weight bytes = 57 / (16*NT)).
#include <algorithm>
#include <cmath>
#include <mutex>

#include "dfmi_core.h"
#include "dfmi_host.h"
#include "dfmi_stream.h"

namespace dfmi {

struct DenseArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int M, K, N;
  int chunks;  // ceil(K / 256)
};

template <typename Tag, int GS, int MT, int NT, bool KFULL>
__global__ __launch_bounds__(kMaxWaves * 64) void qmm_dense_kernel(DenseArgs a) {
  using C = Core<Tag, GS, MT, NT, KFULL>;
  __shared__ __attribute__((aligned(16))) float lds[C::LDS_BYTES / 4];

  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform values in scalar registers, so the chunk loop is a scalar loop
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  const int m_base = blockIdx.y * 16 * MT;

  const typename C::XRows xr = C::x_rows(m_base, a.M, a.K, lane);
  const uint32_t kw = (uint32_t)(a.K / 8);
  const uint32_t kgrp = (uint32_t)(a.K / GS);
  typename C::Rows r;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = min(n0 + t * 16 + (lane & 15), a.N - 1);
    r.wbase[t] = a.w;
    r.sbase[t] = a.s;
    r.bbase[t] = a.b;
    r.woff[t] = (uint32_t)row * kw;
    r.soff[t] = (uint32_t)row * kgrp;
  }

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = zero4();
  // Rotate the K-range of each wavefront by workgroup, so that concurrently
  // running workgroups do not all read the same activation lines at once.
  const int kr = (wave + (int)blockIdx.x) % waves;
  const int c0 = kr * a.chunks / waves;
  const int c1 = (kr + 1) * a.chunks / waves;
  if (c1 > c0) C::run(a.x, xr, r, a.K, c0, c1, acc);

  C::reduce(lds, acc, waves, [&](int t, int mt, int j, int l, float v) {
    const int m = m_base + mt * 16 + 4 * (l >> 4) + j;
    const int n = n0 + t * 16 + (l & 15);
    if (m < a.M && n < a.N) a.y[(int64_t)m * a.N + n] = Num<Tag>::f2h(v);
  });
}

struct DensePlan {
  int MT, NT, waves, chunks, grid_x, grid_y;
  bool kfull;
};

static int plan_dense(int64_t M, int64_t K, int64_t N, const dfmi_qmm_tuning* tune, DensePlan& p) {
  p.MT = M <= 16 ? 1 : 2;
  p.grid_y = M <= 32 ? 1 : (int)((M + 31) / 32);
  p.chunks = (int)((K + kChunkK - 1) / kChunkK);
  p.kfull = (K % kChunkK) == 0;
  int nt = (tune && tune->tiles_per_wave) ? tune->tiles_per_wave
                                          : (N <= 8192 ? 1 : (N <= 32768 ? 2 : 4));
  if (nt != 1 && nt != 2 && nt != 4) {
    set_error("dfmi_qmm: tiles_per_wave must be 1, 2 or 4 (got %d)", nt);
    return DFMI_EINVAL;
  }
  int waves = (tune && tune->waves_per_block) ? tune->waves_per_block : kMaxWaves;
  if (waves < 1 || waves > kMaxWaves) {
    set_error("dfmi_qmm: waves_per_block must be 1..%d (got %d)", kMaxWaves, waves);
    return DFMI_EINVAL;
  }
  p.NT = nt;
  p.waves = std::min(waves, p.chunks);
  p.grid_x = (int)((N + 16 * nt - 1) / (16 * nt));
  return DFMI_OK;
}

template <typename Tag, int GS, int MT, int NT>
static void launch_kf(const DensePlan& p, hipStream_t st, const DenseArgs& a) {
  const dim3 g(p.grid_x, p.grid_y), blk(64 * p.waves);
  if (p.kfull)
    hipLaunchKernelGGL((qmm_dense_kernel<Tag, GS, MT, NT, true>), g, blk, 0, st, a);
  else
    hipLaunchKernelGGL((qmm_dense_kernel<Tag, GS, MT, NT, false>), g, blk, 0, st, a);
}

template <typename Tag, int GS, int MT>
static void launch_mt(const DensePlan& p, hipStream_t st, const DenseArgs& a) {
  if (p.NT == 1) launch_kf<Tag, GS, MT, 1>(p, st, a);
  else if (p.NT == 2) launch_kf<Tag, GS, MT, 2>(p, st, a);
  else launch_kf<Tag, GS, MT, 4>(p, st, a);
}

template <typename Tag, int GS>
static void launch_gs(const DensePlan& p, hipStream_t st, const DenseArgs& a) {
  if (p.MT == 1) launch_mt<Tag, GS, 1>(p, st, a);
  else launch_mt<Tag, GS, 2>(p, st, a);
}

template <typename Tag>
static void launch_tag(int gs, const DensePlan& p, hipStream_t st, const DenseArgs& a) {
  if (gs == 32) launch_gs<Tag, 32>(p, st, a);
  else if (gs == 64) launch_gs<Tag, 64>(p, st, a);
  else launch_gs<Tag, 128>(p, st, a);
}

// ---------------------------------------------------------------------------
// Fast path (Stream main loop): M <= 32, K % 256 == 0, K % (8 * group) == 0.
// A workgroup of 4 wavefronts owns 64 weight rows and a range of the K
// chunks; its wavefronts' partial tiles are summed through LDS.  When the K
// range is split over kp workgroups, each writes its fp32 partial with
// device-coherent stores (agent-scope relaxed atomic stores: write-through,
// no cache flush), waits for them to complete, then bumps the block's counter
// with an atomic RMW; the workgroup that takes the counter to kp sums the kp
// partials in split order (device-coherent loads) and writes y, so the result
// does not depend on arrival order.  No device-scope fence is needed because
// no plain store is published across workgroups.

constexpr size_t kCounterBytes = 65536;
constexpr int kMaxCounters = (int)(kCounterBytes / 4);
constexpr int kMaxSeg = 4;  // weight matrices of one shared-activation launch

struct StreamArgs {
  const uint16_t* x;
  float* partials;     // [kp][M][pstride] fp32 (kp > 1)
  uint32_t* counters;  // [n_blocks] (kp > 1), zero between calls
  int M, K;
  int chunks;
  int kp;
  int n_blocks;
  int xcd_map;
  int pstride;  // columns of a partial row: 64 x (n_blocks - whole)
  int whole;    // blocks [0, whole) run unsplit, one workgroup each; the rest kp-way split
};

// One weight matrix of a launch: the launch's blocks blk0 .. blk0 +
// ceil(N / 64) - 1 are its row blocks; its partial columns are
// 64 blk0 + row.
struct StreamSeg {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int N;
  int blk0;
  const uint32_t* t;  // [K/GS][N] (scale, bias) pairs (pair-streaming kernels), or null
};

struct StreamSegs {
  StreamSeg seg[kMaxSeg];
  int nseg;
  // [K/GS][sum of N] pair table of all the matrices side by side (each
  // segment's own t then unused), or null: qmm_stream_fused_kernel
  const uint32_t* fused;
  // the row length (in pairs) of the table every segment's t points into
  // (each t its matrix's column slice of a wider table: column 0 of the
  // slice), or 0 when each t is its matrix's own [K/GS][N] table
  uint32_t tn;
};

// workgroup L -> (block nb, K split kpi of kpw).  Workgroups [0, whole) take
// blocks [0, whole) whole; the rest take the kp splits of the later blocks
// (whole is a multiple of 8, so L - whole keeps L's XCD).
__device__ inline void stream_unit_of(int L, int whole, int kp, int xcd_map, int& nb, int& kpi,
                                      int& kpw) {
  if (L < whole) {
    nb = L;
    kpi = 0;
    kpw = 1;
    return;
  }
  L -= whole;
  kpw = kp;
  if (xcd_map) {
    // round-robin dispatch sends consecutive workgroup ids to different XCDs
    // (id & 7): give the kp splits of one block ids of one residue so that,
    // where placement follows it, the block's partials and counter stay in
    // one L2 (correctness does not depend on it: the exchange is agent-scope
    // atomics)
    const int xcd = L & 7, j = L >> 3;
    const int nbl = j / kp;
    kpi = j - nbl * kp;
    nb = nbl * 8 + xcd;
  } else {
    nb = L / kp;
    kpi = L - nb * kp;
  }
  nb += whole;
}

// Block nb (of matrix g), K split kpi of kp.  TSB: scales and biases come
// from g.t, the pair table, one step at a time.  RW = 2: 128-row blocks, two
// row groups of WV / 2 wavefronts.
template <typename Tag, int GS, int MT, int WV, int BITS, int SBPC, bool TSB, int RW>
__device__ __forceinline__ void qmm_stream_body(const StreamArgs& a, const StreamSeg& g, int nb,
                                                int kpi, int kp, uint32_t tn = 0,
                                                uint32_t tc = 0) {
  using S = Stream<Tag, GS, MT, WV, SBPC, BITS, RW, TSB>;
  constexpr int kThreads = 64 * WV;
  typename S::Ctx cx;
  cx.x = buffer_rsrc(a.x, (uint32_t)a.M * (uint32_t)a.K * 2u);
  cx.w = buffer_rsrc(g.w, (uint32_t)g.N * (uint32_t)(a.K / 8 * BITS));
  cx.s = buffer_rsrc(g.s, (uint32_t)g.N * (uint32_t)(a.K / GS) * 2u);
  cx.b = buffer_rsrc(g.b, (uint32_t)g.N * (uint32_t)(a.K / GS) * 2u);
  // TSB: g.t is this matrix's [K/GS][N] pair table, or (tn > 0) a table of
  // tn columns holding it from column tc on
  if constexpr (TSB)
    cx.t = buffer_rsrc(g.t, (tn ? tn : (uint32_t)g.N) * (uint32_t)(a.K / GS) * 4u);
  cx.K = a.K;
  cx.M = a.M;
  cx.N = g.N;
  cx.groups = a.K / GS;
  cx.n0 = (nb - g.blk0) * S::NB;
  cx.lane = threadIdx.x & 63;
  cx.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  cx.dense();
  cx.tn = tn;
  cx.tc = tc;
  const int c0 = (int)((int64_t)kpi * a.chunks / kp);
  const int c1 = (int)((int64_t)(kpi + 1) * a.chunks / kp);
  f32x4 acc[S::NT][MT];
#pragma unroll
  for (int t = 0; t < S::NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = zero4();
  S::run(cx, c0, c1, acc);

  // sum the partial tiles of each row group's KW wavefronts through LDS (the
  // stages are free: every DMA has landed and every wavefront is past its
  // last LDS read), in k-slice order
  __syncthreads();
  float* red = reinterpret_cast<float*>(dfmi_smem);
  {
    float* mine = red + cx.wave * S::RED_FLOATS;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) mine[((t * MT + mt) * 4 + j) * 64 + cx.lane] = acc[t][mt][j];
  }
  __syncthreads();
  constexpr int PER = RW * S::RED_FLOATS / kThreads;
  float v[PER];
  int mi[PER], ni[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = q * kThreads + threadIdx.x;
    const int rg = e / S::RED_FLOATS, eo = e % S::RED_FLOATS;
    const float* rr = red + rg * S::KW * S::RED_FLOATS + eo;
    float sum = rr[0];
#pragma unroll
    for (int k = 1; k < S::KW; ++k) sum += rr[k * S::RED_FLOATS];
    v[q] = sum;
    const int l = eo & 63, j = (eo >> 6) & 3, tm = eo >> 8;
    ni[q] = cx.n0 + kStreamRows * rg + (tm / MT) * 16 + (l & 15);
    mi[q] = (tm % MT) * 16 + 4 * (l >> 4) + j;
  }
  if (kp == 1) {
#pragma unroll
    for (int q = 0; q < PER; ++q)
      if (mi[q] < a.M && ni[q] < g.N) g.y[(int64_t)mi[q] * g.N + ni[q]] = Num<Tag>::f2h(v[q]);
    return;
  }
  // split blocks only (nb >= whole) have partial columns: block nb's are
  // NB (nb - whole) + row, so this matrix's start at NB (blk0 - whole)
  float* part = a.partials + (int64_t)kpi * a.M * a.pstride + (int64_t)(g.blk0 - a.whole) * S::NB;
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (mi[q] < a.M && ni[q] < g.N)
      __hip_atomic_store(part + (int64_t)mi[q] * a.pstride + ni[q], v[q], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  int* s_last = reinterpret_cast<int*>(dfmi_smem);  // red[0], already consumed
  stage_barrier<0>();  // every partial store of the workgroup has completed
  if (threadIdx.x == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&a.counters[nb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = (prev == (unsigned)(kp - 1)) ? 1 : 0;
  }
  stage_barrier<0>();
  if (!*s_last) return;
  // Sum the kp partials of this thread's outputs in split order.  The
  // device-coherent loads of eight splits x PER outputs are issued together
  // (one memory round trip per eight splits, not one per load).
  float sum[PER];
  int64_t off[PER];
  bool ok[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    sum[q] = 0.f;
    ok[q] = mi[q] < a.M && ni[q] < g.N;
    off[q] = ok[q] ? (int64_t)mi[q] * a.pstride + (int64_t)(g.blk0 - a.whole) * S::NB + ni[q] : 0;
  }
  const int64_t split = (int64_t)a.M * a.pstride;
  for (int q0 = 0; q0 < kp; q0 += 8) {
    // unconditional loads (a split past kp re-reads the last one and is
    // dropped), so the block is straight-line code with one wait
    float t[8][PER];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t base = (int64_t)min(q0 + j, kp - 1) * split;
#pragma unroll
      for (int q = 0; q < PER; ++q)
        t[j][q] = __hip_atomic_load(a.partials + base + off[q], __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < PER; ++q) sum[q] += (q0 + j < kp) ? t[j][q] : 0.f;
  }
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (ok[q]) g.y[(int64_t)mi[q] * g.N + ni[q]] = Num<Tag>::f2h(sum[q]);
  if (threadIdx.x == 0)
    __hip_atomic_exchange(&a.counters[nb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct StreamPlan {
  int MT, WV, kp, chunks, n_blocks, grid_x, xcd_map, lds;
  int whole;  // blocks run unsplit ahead of the kp-way split ones
  int bits;  // 4 or 8
  int sbpc;  // scale / bias window pieces (8-bit with 8 wavefronts: 8, to fit LDS)
  int tsb;   // the pair-streaming kernel runs this plan when the pair tables are given
  int rw;    // 64-row groups per block: 1, or 2 (128-row pair-streaming blocks)
  size_t ws_bytes;
};

constexpr int kCUs = 256;  // MI355X compute units
// 128-row pair-streaming blocks as the automatic choice where every matrix
// is a whole number of them
constexpr bool kAutoRows128 = true;

// Shapes with a pair-streaming plan: 4-bit, gs 64 / 128, one or two
// activation blocks (M <= 32), whole 256-k steps (and a split's K range
// within the window of the kernel that runs the same plan without pair
// tables).
static bool tsb_shape(int64_t M, int64_t K, int64_t N, int gs, int bits) {
  return bits == 4 && (gs == 64 || gs == 128) && M >= 1 && M <= 32 && K % 256 == 0 &&
         K % (8 * gs) == 0 && (N + kStreamRows - 1) / kStreamRows <= kMaxCounters;
}

// The matrices of a launch in both block sizes: 64-row blocks, and 128-row
// blocks when every matrix is a whole number of them (else 0).
struct StreamGeo {
  int nb64;
  int nb128;
};

static StreamGeo geo_of(const int64_t* Ns, int nseg) {
  StreamGeo g{0, 0};
  bool even = true;
  for (int i = 0; i < nseg; ++i) {
    g.nb64 += (int)((Ns[i] + kStreamRows - 1) / kStreamRows);
    even = even && Ns[i] % (2 * kStreamRows) == 0;
    g.nb128 += (int)(Ns[i] / (2 * kStreamRows));
  }
  if (!even) g.nb128 = 0;
  return g;
}

// The automatic plan of a pair-streaming shape, 256-k steps.  rw = 1: 64-row
// blocks, 4 wavefronts, 51 KB, three workgroups per CU; rw = 2: 128-row
// blocks (two row groups sharing each activation stage, half the activation
// requests per weight byte), 8 wavefronts, 78 KB, two per CU.  With P
// workgroups resident per CU (S = 256 P slots), measured on MI355X:
//  * >= S blocks: whole blocks; the last partial round's blocks (at most a
//    quarter round) split over every slot;
//  * w = blocks / 256 in 1 .. P-1: w whole blocks per CU and the rest split
//    into at most P - w pieces per CU, so every CU streams the same bytes
//    (5120 x 34816 at rw 1: 27.3 us, all whole 31.2 us);
//  * fewer than 256: K split so that one workgroup per CU runs
//    (kp = 256 / blocks; 5120 x 5120 at rw 1: kp 3 9.0 us, kp 9 12.3 us;
//    4096 x 24576 at rw 2: kp 1 15.7 us, kp 2 19.2 us): more, shorter
//    splits pay more fills and exchanges than they gain.
// The same plan (in 64-row blocks: each 128-row block as two) runs on the
// window kernel when no pair tables are given (80 KB workgroups, two per
// CU), so both give bit-identical results.
static void plan_tsb(int64_t K, const StreamGeo& geo, int gs, int rw, int kp_force, int mt,
                     StreamPlan& p) {
  p.bits = 4;
  p.MT = mt;
  p.rw = rw;
  p.WV = 4 * rw;
  p.tsb = 1;
  p.sbpc = kSbPieces;
  p.n_blocks = rw == 2 ? geo.nb128 : geo.nb64;
  p.chunks = (int)(K / 256);
  const int per_cu = rw == 2 ? 2 : 3;
  const int slots = kCUs * per_cu;
  const int max_chunks = sb_max_groups(kSbPieces) / (256 / gs);  // window of a split
  const int kmin = (p.chunks + max_chunks - 1) / max_chunks;
  const int nb = p.n_blocks;
  p.whole = 0;
  p.kp = kmin;
  if (kp_force > 0) {
    p.kp = std::max(kmin, std::min(kp_force, p.chunks));
  } else if (kmin == 1 && nb >= slots) {
    const int left = nb % slots;
    if (left > 0 && 4 * left <= slots) {
      p.whole = nb - left;
      p.kp = std::max(1, std::min((int)std::lround((double)slots / left), p.chunks));
    }
  } else if (kmin == 1 && nb >= kCUs) {
    const int w = nb / kCUs;  // whole blocks per CU, 1 .. per_cu - 1
    const int left = nb - w * kCUs;
    p.kp = left > 0 ? std::max(1, std::min((per_cu - w) * kCUs / left, p.chunks)) : 1;
    p.whole = p.kp > 1 ? w * kCUs : 0;
    if (!p.whole) p.kp = 1;
  } else if (nb < kCUs) {
    const int kp = std::max(1, kCUs / nb);
    p.kp = std::max(kmin, std::min(kp, std::max(1, p.chunks / 2)));
    // two activation blocks (two stages, one in flight): raise the split
    // toward two workgroups per CU while every split keeps >= 8 steps
    // (27B-class down projection at M = 32: 6 splits 23.5 us vs 3 splits
    // 25.7 us; o: 3 splits 12.0 us, 6 splits 12.7 us)
    if (mt == 2) p.kp = std::max(p.kp, std::min(2 * kCUs / nb, p.chunks / 8));
  }
  p.xcd_map = ((nb - p.whole) % 8 == 0) ? 1 : 0;
}

// A 128-row plan as the equivalent 64-row plan (each block as two with the
// same K splits, so every output is summed in the same order): what the
// window kernel runs when the pair tables are missing.
static void plan_as_rows64(StreamPlan& p) {
  if (p.rw != 2) return;
  p.rw = 1;
  p.WV = 4;
  p.n_blocks *= 2;
  p.whole *= 2;
  p.grid_x = p.whole + (p.n_blocks - p.whole) * p.kp;
  p.xcd_map = ((p.n_blocks - p.whole) % 8 == 0) ? 1 : 0;
}

// Scale / bias window pieces of the streaming kernel: 16, except for 8-bit
// weights with 8 wavefronts, whose twice-as-long weight stages leave LDS for
// an 8-piece window only (16 + 48 + 96 KB = 160 KB).
static int stream_sb_pieces(int bits, int wv) { return bits == 8 && wv == 8 ? 8 : kSbPieces; }

// 8 wavefronts (512-k steps, two wavefronts per SIMD, one workgroup per CU)
// when K allows and the grid fits on the 256 CUs at once; else 4 wavefronts
// (two workgroups per CU).
static int stream_waves(int64_t M, int64_t K, int grid) {
  return (M <= 16 && K % 512 == 0 && grid <= 256) ? 8 : 4;
}

// Ns / nseg: the matrices of a shared-activation launch (N = their 64-row
// blocks' columns); nullptr: one matrix of N rows.
static int plan_stream(int64_t M, int64_t K, int64_t N, int gs, int bits,
                       const dfmi_qmm_tuning* tune, StreamPlan& p, const int64_t* Ns = nullptr,
                       int nseg = 1) {
  p.tsb = 0;
  p.rw = 1;
  const int64_t one[1] = {N};
  const StreamGeo geo = geo_of(Ns ? Ns : one, Ns ? nseg : 1);
  const int rows = tune ? tune->rows_per_block : 0;
  if (rows != 0 && rows != 64 && rows != 128) {
    set_error("dfmi_qmm: rows_per_block must be 0, 64 or 128 (got %d)", rows);
    return DFMI_EINVAL;
  }
  const bool waves = tune && tune->waves_per_block > 0;
  const bool tsb = tsb_shape(M, K, N, gs, bits);
  const int mt = M <= 16 ? 1 : 2;  // activation blocks of 16 rows
  if (rows == 128 && (!tsb || !geo.nb128 || waves || mt == 2)) {
    set_error("dfmi_qmm: 128-row blocks need a pair-streaming shape (4-bit, gs 64 / 128, "
              "M <= 16, K %% 256 == 0, every N a multiple of 128) and automatic wavefronts");
    return DFMI_EINVAL;
  }
  if (tsb && !waves) {
    const int kp_force = tune ? tune->k_splits : 0;
    // 128-row blocks where a workgroup streams 8 steps or more on average (measured
    // on MI355X: the second row group's stage fill pays off over long
    // ranges -- 5120 x 34816 24.5 vs 26.7 us, 17408 x 5120 15.6 vs 17.2 us,
    // 5120 x 151936 95.5 vs 102.7 us -- and loses on short ones: 5120 x
    // 5120 9.6 vs 9.0 us, 4096 x 4096 8.7 vs 7.9 us)
    // (two activation blocks: 64-row blocks only, two stages of 25 KB, three
    // workgroups per CU)
    int rw = rows == 128 ? 2 : 1;
    if (rows == 0 && geo.nb128 && kAutoRows128 && mt == 1) {
      StreamPlan q;
      plan_tsb(K, geo, gs, 2, kp_force, 1, q);
      const int grid = q.whole + (q.n_blocks - q.whole) * q.kp;
      if ((int64_t)q.n_blocks * q.chunks >= 8ll * grid) rw = 2;
    }
    plan_tsb(K, geo, gs, rw, kp_force, mt, p);
    p.grid_x = p.whole + (p.n_blocks - p.whole) * p.kp;
    p.ws_bytes = p.kp > 1 ? kCounterBytes + (size_t)p.kp * (size_t)M *
                                                 (size_t)(p.n_blocks - p.whole) *
                                                 (size_t)(kStreamRows * p.rw) * 4u
                          : 0;
    return DFMI_OK;
  }
  p.bits = bits;
  p.MT = M <= 16 ? 1 : 2;
  p.n_blocks = (int)((N + kStreamRows - 1) / kStreamRows);
  int kp;
  if (tune && tune->k_splits > 0) {
    kp = tune->k_splits;
  } else {
    // one workgroup per CU on 256 CUs, at least 4 steps of 256 k per split
    // (every split pays a pipeline fill and the partial-sum epilogue)
    kp = (int)std::lround(256.0 / (double)p.n_blocks);
    kp = std::max(1, std::min(kp, (int)(K / 1024)));
    // two 4-bit activation blocks: two 80 KB workgroups share a CU, so up to
    // 512 workgroups run at once; raise the split toward that while every
    // split keeps at least 8 steps (27B-class down projection at M = 32:
    // 6 splits 21.5 us vs 3 splits 25.2 us)
    if (p.MT == 2 && bits == 4)
      kp = std::max(kp, std::min(512 / p.n_blocks, (int)(K / 2048)));
  }
  p.kp = std::max(1, std::min(kp, (int)(K / 256)));
  if (p.n_blocks > kMaxCounters) p.kp = 1;
  p.WV = stream_waves(M, K, p.n_blocks * p.kp);
  // 8-bit weights: 8 wavefronts take 160 KB (one workgroup per CU), 4 in
  // two stages 80 KB (two per CU).  An unsplit 8-wavefront grid that leaves
  // CUs idle runs as 4 wavefronts with its K split toward 512 workgroups
  // instead (4096x12288: 15.2 us vs 20.1 us).
  if (!(tune && tune->k_splits > 0) && bits == 8 && p.MT == 1 && p.WV == 8 && p.kp == 1 &&
      p.n_blocks < 256) {
    p.WV = 4;
    p.kp = std::max(1, std::min(512 / p.n_blocks, (int)(K / 1024)));
  }
  if (tune && (tune->waves_per_block == 4 || tune->waves_per_block == 8) &&
      (tune->waves_per_block == 4 || (M <= 16 && K % 512 == 0)))
    p.WV = tune->waves_per_block;
  p.chunks = (int)(K / (64 * p.WV));
  p.kp = std::min(p.kp, p.chunks);
  // a split's K range fits one scale / bias window
  p.sbpc = stream_sb_pieces(bits, p.WV);
  const int max_chunks = sb_max_groups(p.sbpc) / (64 * p.WV / gs);
  p.kp = std::max(p.kp, (p.chunks + max_chunks - 1) / max_chunks);
  p.whole = 0;
  p.xcd_map = (p.n_blocks % 8 == 0) ? 1 : 0;
  // A grid a little past whole rounds of the workgroups that run at once
  // (two per CU with 4 wavefronts, one with 8) would end with a round of a
  // few whole blocks, as long as a full round: a workgroup streams at a
  // latency-bound rate whatever the others do (27B-class gate/up, 544 blocks
  // on 512 slots: 32.8 us, 512 blocks: 24.9 us).  So the whole rounds run
  // unsplit and the leftover blocks (at most a quarter round) are split
  // finely enough to spread over every slot.
  const int slots = p.WV == 8 ? 256 : 512;
  if (!(tune && tune->k_splits > 0) && p.kp == 1 && p.n_blocks > slots &&
      p.n_blocks <= kMaxCounters) {
    const int whole = (p.n_blocks / slots) * slots;
    const int left = p.n_blocks - whole;
    if (left > 0 && 4 * left <= slots) {
      p.whole = whole;
      p.kp = std::max(1, std::min((int)std::lround((double)slots / left), p.chunks));
      p.xcd_map = (left % 8 == 0) ? 1 : 0;
    }
  }
  p.grid_x = p.whole + (p.n_blocks - p.whole) * p.kp;
  // forced plans of pair-streaming shapes may still run the pair kernel
  p.tsb = (tsb_shape(M, K, N, gs, bits) && p.WV == 4) ? 1 : 0;
  p.ws_bytes = p.kp > 1 ? kCounterBytes + (size_t)p.kp * (size_t)M *
                                               (size_t)(p.n_blocks - p.whole) * kStreamRows * 4u
                        : 0;
  return DFMI_OK;
}

// The arguments as scalars, not a by-value struct, so that they are
// preloaded into SGPRs at wave start (-amdgpu-kernarg-preload-count): the
// hardware preloads 14 dwords on gfx950, so everything the first DMA needs
// comes first (x, w, t, s, b, a packed word M | xcd_map << 6 | kp << 7 |
// chunks << 16, N, whole, the pair table's row length tn (0: N); the block
// count and K follow from N and chunks) and the outputs and split-K
// workspace, first needed in the epilogue, last.  (With M, K, N ... after
// the eight pointers a workgroup waited for one scalar-load round trip
// before its first DMA.)
template <typename Tag, int GS, int MT, int WV, int BITS, int SBPC, bool TSB, int RW>
__global__ __launch_bounds__(64 * WV) void qmm_stream_kernel(
    const uint16_t* x, const uint32_t* w, const uint32_t* t, const uint16_t* s,
    const uint16_t* b, uint32_t p0, int N, int whole, uint32_t tn, uint16_t* y, float* partials,
    uint32_t* counters) {
  using S = Stream<Tag, GS, MT, WV, SBPC, BITS, RW, TSB>;
  const int M = (int)(p0 & 63u), xcd_map = (int)((p0 >> 6) & 1u), kp = (int)((p0 >> 7) & 511u);
  const int chunks = (int)(p0 >> 16);
  const int n_blocks = (N + S::NB - 1) / S::NB;
  int nb, kpi, kpw;
  stream_unit_of(blockIdx.x, whole, kp, xcd_map, nb, kpi, kpw);
  if (nb >= n_blocks) return;  // uniform, before any barrier
  qmm_stream_body<Tag, GS, MT, WV, BITS, SBPC, TSB, RW>(
      StreamArgs{x, partials, counters, M, chunks * S::CK, chunks, kp, n_blocks, xcd_map,
                 kStreamRows * RW * (n_blocks - whole), whole},
      StreamSeg{w, s, b, y, N, 0, t}, nb, kpi, kpw, tn, 0u);
}

// Several weight matrices over the same activations (q / k / v, gate / up):
// their row blocks form one grid.
template <typename Tag, int GS, int MT, int WV, int BITS, int SBPC, bool TSB, int RW>
__global__ __launch_bounds__(64 * WV) void qmm_stream_multi_kernel(StreamArgs a, StreamSegs m) {
  int nb, kpi, kpw;
  stream_unit_of(blockIdx.x, a.whole, a.kp, a.xcd_map, nb, kpi, kpw);
  if (nb >= a.n_blocks) return;  // uniform, before any barrier
  // the matrix holding block nb (constant indices: the table stays in SGPRs)
  StreamSeg g = m.seg[0];
#pragma unroll
  for (int i = 1; i < kMaxSeg; ++i)
    if (i < m.nseg && nb >= m.seg[i].blk0) g = m.seg[i];
  qmm_stream_body<Tag, GS, MT, WV, BITS, SBPC, TSB, RW>(a, g, nb, kpi, kpw, m.tn, 0u);
}

// Two or three matrices over the same activations whose pair tables sit side
// by side in one [K/GS][N0 + N1 + N2] table (pair streaming only).  Every
// value the workgroup needs before its first DMA is in the first 14 argument
// dwords, which the hardware preloads into SGPRs: the activations, the
// table, the weights, and three packed words (M | kp << 6 | xcd_map << 13 |
// chunks << 16; whole | N2 << 16; N0 | N1 << 16).  The outputs and the
// split-K workspace are read from the kernel arguments when the epilogue
// needs them.  (qmm_stream_multi_kernel instead loads its segment table
// before the first DMA: ~0.6-0.9 us per launch on MI355X.)
template <typename Tag, int GS, int MT, int WV, int RW>
__global__ __launch_bounds__(64 * WV) void qmm_stream_fused_kernel(
    const uint16_t* x, const uint32_t* t, const uint32_t* w0, const uint32_t* w1,
    const uint32_t* w2, uint32_t p0, uint32_t p1, uint32_t p2, uint16_t* y0, uint16_t* y1,
    uint16_t* y2, uint32_t* counters, float* partials, int pstride) {
  constexpr int NB = kStreamRows * RW;
  const int M = (int)(p0 & 63u), kp = (int)((p0 >> 6) & 127u), xcd_map = (int)((p0 >> 13) & 1u);
  const int chunks = (int)(p0 >> 16);
  const int whole = (int)(p1 & 0xFFFFu), N2 = (int)(p1 >> 16);
  const int N0 = (int)(p2 & 0xFFFFu), N1 = (int)(p2 >> 16);
  const int b1 = (N0 + NB - 1) / NB, b2 = b1 + (N1 + NB - 1) / NB;
  const int n_blocks = b2 + (N2 + NB - 1) / NB;
  int nb, kpi, kpw;
  stream_unit_of(blockIdx.x, whole, kp, xcd_map, nb, kpi, kpw);
  if (nb >= n_blocks) return;  // uniform, before any barrier
  const bool in1 = nb >= b1, in2 = nb >= b2;  // segment 1 / 2 (uniform)
  StreamSeg g;
  g.w = in2 ? w2 : (in1 ? w1 : w0);
  g.s = nullptr;  // pair streaming: no scale / bias window
  g.b = nullptr;
  g.y = in2 ? y2 : (in1 ? y1 : y0);
  g.N = in2 ? N2 : (in1 ? N1 : N0);
  g.blk0 = in2 ? b2 : (in1 ? b1 : 0);
  g.t = t;
  const uint32_t tc = in2 ? (uint32_t)(N0 + N1) : (in1 ? (uint32_t)N0 : 0u);
  qmm_stream_body<Tag, GS, MT, WV, 4, kSbPieces, true, RW>(
      StreamArgs{x, partials, counters, M, chunks * 256, chunks, kp, n_blocks, xcd_map, pstride,
                 whole},
      g, nb, kpi, kpw, (uint32_t)(N0 + N1 + N2), tc);
}

// The fused kernel takes the launch: two or three matrices, each N < 2^16,
// and the plan's values fit their packed fields.
// (Every matrix's N a multiple of 4 as well: each lane's 16-byte load of
// pairs then starts on a 16-byte boundary of the combined table.)
static bool fused_fits(const StreamSegs& m, int whole, int kp, int chunks, int M) {
  if (!m.fused || m.nseg < 2 || m.nseg > 3) return false;
  for (int i = 0; i < m.nseg; ++i)
    if (m.seg[i].N >= 65536 || m.seg[i].N % 4) return false;
  return whole < 65536 && kp < 128 && chunks < 65536 && M < 64;
}

// Every matrix of m carries its pair table (or they share a fused one).
static bool segs_have_pairs(const StreamSegs& m) {
  if (m.fused) return true;
  for (int i = 0; i < m.nseg; ++i)
    if (m.seg[i].N > 0 && !m.seg[i].t) return false;
  return true;
}

template <typename Tag, int GS, int MT, int WV, int BITS, bool TSB, int RW>
static void launch_stream_k(const StreamPlan& p, hipStream_t st, const StreamArgs& a,
                            const StreamSegs& m) {
  constexpr int SBPC = BITS == 8 && WV == 8 ? 8 : kSbPieces;  // = stream_sb_pieces(BITS, WV)
  const int lds = Stream<Tag, GS, MT, WV, SBPC, BITS, RW, TSB>::LDS_BYTES;
  if (m.nseg == 1) {
    const StreamSeg& g = m.seg[0];
    // (the packed fields hold every plan: M <= 32, kp < 512, chunks < 2^16;
    // launch_streaming checks them)
    const uint32_t p0 = (uint32_t)a.M | ((uint32_t)a.xcd_map << 6) | ((uint32_t)a.kp << 7) |
                        ((uint32_t)a.chunks << 16);
    hipLaunchKernelGGL((qmm_stream_kernel<Tag, GS, MT, WV, BITS, SBPC, TSB, RW>), dim3(p.grid_x),
                       dim3(64 * WV), lds, st, a.x, g.w, g.t, g.s, g.b, p0, g.N, a.whole, m.tn,
                       g.y, a.partials, a.counters);
  } else {
    if constexpr (TSB && BITS == 4 && GS >= 64) {
      if (m.fused) {  // fused_fits() held when the plan was made
        const uint32_t p0 = (uint32_t)a.M | ((uint32_t)a.kp << 6) | ((uint32_t)a.xcd_map << 13) |
                            ((uint32_t)a.chunks << 16);
        const uint32_t p1 = (uint32_t)a.whole | ((uint32_t)(m.nseg > 2 ? m.seg[2].N : 0) << 16);
        const uint32_t p2 = (uint32_t)m.seg[0].N | ((uint32_t)m.seg[1].N << 16);
        hipLaunchKernelGGL((qmm_stream_fused_kernel<Tag, GS, MT, WV, RW>), dim3(p.grid_x),
                           dim3(64 * WV), lds, st, a.x, m.fused, m.seg[0].w, m.seg[1].w,
                           m.nseg > 2 ? m.seg[2].w : m.seg[1].w, p0, p1, p2, m.seg[0].y,
                           m.seg[1].y, m.nseg > 2 ? m.seg[2].y : m.seg[1].y, a.counters,
                           a.partials, a.pstride);
        return;
      }
    }
    hipLaunchKernelGGL((qmm_stream_multi_kernel<Tag, GS, MT, WV, BITS, SBPC, TSB, RW>),
                       dim3(p.grid_x), dim3(64 * WV), lds, st, a, m);
  }
}

// The pair-streaming kernel when the plan allows it and every matrix has its
// pair table (4-bit, gs 64 / 128, one activation block; 4 wavefronts and
// 64-row blocks, or 8 wavefronts and 128-row blocks).  The launcher has
// already turned a 128-row plan into its 64-row equivalent when the tables
// are missing.
template <typename Tag, int GS, int MT, int WV, int BITS>
static void launch_stream_t(const StreamPlan& p, hipStream_t st, const StreamArgs& a,
                            const StreamSegs& m) {
  if constexpr (BITS == 4 && GS >= 64 && MT == 1) {
    if (p.tsb && p.rw == 2 && WV == 8) {
      launch_stream_k<Tag, GS, MT, 8, BITS, true, 2>(p, st, a, m);
      return;
    }
  }
  if constexpr (BITS == 4 && GS >= 64 && WV == 4) {
    if (p.tsb && p.rw == 1 && segs_have_pairs(m)) {
      launch_stream_k<Tag, GS, MT, WV, BITS, true, 1>(p, st, a, m);
      return;
    }
  }
  launch_stream_k<Tag, GS, MT, WV, BITS, false, 1>(p, st, a, m);
}

template <typename Tag, int GS, int BITS>
static void launch_stream_bits(const StreamPlan& p, hipStream_t st, const StreamArgs& a,
                               const StreamSegs& m) {
  if (p.MT == 1) {
    if (p.WV == 8) launch_stream_t<Tag, GS, 1, 8, BITS>(p, st, a, m);
    else launch_stream_t<Tag, GS, 1, 4, BITS>(p, st, a, m);
  } else {
    launch_stream_t<Tag, GS, 2, 4, BITS>(p, st, a, m);
  }
}

template <typename Tag, int GS>
static void launch_stream_gs(const StreamPlan& p, hipStream_t st, const StreamArgs& a,
                             const StreamSegs& m) {
  if (p.bits == 8) launch_stream_bits<Tag, GS, 8>(p, st, a, m);
  else launch_stream_bits<Tag, GS, 4>(p, st, a, m);
}

template <typename Tag>
static void launch_stream(int gs, const StreamPlan& p, hipStream_t st, const StreamArgs& a,
                          const StreamSegs& m) {
  if (gs == 32) launch_stream_gs<Tag, 32>(p, st, a, m);
  else if (gs == 64) launch_stream_gs<Tag, 64>(p, st, a, m);
  else launch_stream_gs<Tag, 128>(p, st, a, m);
}

// Dynamic LDS above 64 KiB needs the per-kernel attribute raised once.
template <typename Tag, int GS, int MT, int WV, int BITS>
static void allow_lds_t() {
  constexpr int SBPC = BITS == 8 && WV == 8 ? 8 : kSbPieces;
  constexpr int lds = Stream<Tag, GS, MT, WV, SBPC, BITS>::LDS_BYTES;
  (void)hipFuncSetAttribute(
      reinterpret_cast<const void*>(&qmm_stream_kernel<Tag, GS, MT, WV, BITS, SBPC, false, 1>),
      hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  (void)hipFuncSetAttribute(
      reinterpret_cast<const void*>(
          &qmm_stream_multi_kernel<Tag, GS, MT, WV, BITS, SBPC, false, 1>),
      hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if constexpr (BITS == 4 && GS >= 64 && MT == 1 && WV == 8) {
    constexpr int lds2 = Stream<Tag, GS, MT, 8, kSbPieces, 4, 2, true>::LDS_BYTES;
    (void)hipFuncSetAttribute(
        reinterpret_cast<const void*>(&qmm_stream_kernel<Tag, GS, 1, 8, 4, kSbPieces, true, 2>),
        hipFuncAttributeMaxDynamicSharedMemorySize, lds2);
    (void)hipFuncSetAttribute(
        reinterpret_cast<const void*>(
            &qmm_stream_multi_kernel<Tag, GS, 1, 8, 4, kSbPieces, true, 2>),
        hipFuncAttributeMaxDynamicSharedMemorySize, lds2);
  }
}

template <typename Tag, int GS>
static void allow_lds_gs() {
  allow_lds_t<Tag, GS, 1, 4, 4>();
  allow_lds_t<Tag, GS, 1, 8, 4>();
  allow_lds_t<Tag, GS, 2, 4, 4>();
  allow_lds_t<Tag, GS, 1, 4, 8>();
  allow_lds_t<Tag, GS, 1, 8, 8>();
  allow_lds_t<Tag, GS, 2, 4, 8>();
}

static void allow_lds_all() {
  // once per process (thread-safe static initialisation); the attribute
  // calls are idempotent
  static const bool done = [] {
    allow_lds_gs<BF16, 32>();
    allow_lds_gs<BF16, 64>();
    allow_lds_gs<BF16, 128>();
    allow_lds_gs<F16, 32>();
    allow_lds_gs<F16, 64>();
    allow_lds_gs<F16, 128>();
    return true;
  }();
  (void)done;
}

static int validate_qmm(int x_dtype, int64_t M, int64_t K, int64_t N, int gs, int bits) {
  if (x_dtype != DFMI_BF16 && x_dtype != DFMI_F16) {
    set_error("dfmi_qmm: x dtype %d unsupported (bf16 or f16)", x_dtype);
    return DFMI_EINVAL;
  }
  if (bits != 4 && bits != 8) {
    set_error("dfmi_qmm: bits=%d unsupported (4 or 8)", bits);
    return DFMI_EINVAL;
  }
  if (gs != 32 && gs != 64 && gs != 128) {
    set_error("dfmi_qmm: group_size=%d unsupported (32, 64, 128)", gs);
    return DFMI_EINVAL;
  }
  if (M < 0 || N < 0 || K < 32 || K % 32 || K % gs) {
    set_error("dfmi_qmm: bad shape M=%lld K=%lld N=%lld gs=%d", (long long)M, (long long)K,
              (long long)N, gs);
    return DFMI_EINVAL;
  }
  if (M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31) ||
      N * (K * bits / 32) > 0xFFFFFFFFll) {
    set_error("dfmi_qmm: shape too large M=%lld K=%lld N=%lld", (long long)M, (long long)K,
              (long long)N);
    return DFMI_EINVAL;
  }
  return DFMI_OK;
}

}  // namespace dfmi

using namespace dfmi;

// Automatic choice (measured on MI355X): the streaming kernel is faster on
// every shape it takes; the general kernel covers the rest (M > 32, K not a
// multiple of 256 or of 8 groups, weights over 2 GiB).
static bool use_stream(int64_t M, int64_t K, int64_t N, int gs, int bits,
                       const dfmi_qmm_tuning* tune) {
  const int path = tune ? tune->path : 0;
  if (bits != 4 && bits != 8) return false;
  if (path == 1) return false;
  // more blocks than split counters run unsplit: the whole K in one scale
  // window (8-bit: the smaller window of its plans)
  const int sbpc = bits == 8 ? 8 : kSbPieces;
  return stream_eligible(M, K, N, gs, bits) &&
         ((N + kStreamRows - 1) / kStreamRows <= kMaxCounters || K / gs <= sb_max_groups(sbpc));
}

// tuning.path: 0 automatic, 1 general kernel, 2 streaming kernel
static bool valid_path(const dfmi_qmm_tuning* tune) {
  return !tune || (tune->path >= 0 && tune->path <= 2);
}

// Everything a streaming launch needs except the activations, the outputs
// and the stream: the plan, the kernel arguments and the matrices.
struct StreamLaunch {
  StreamPlan p;
  StreamArgs a;
  StreamSegs m;
  int x_dtype;
  int gs;
};

// Plan the streaming kernel over the matrices of segs (their row blocks one
// grid of n_cols / 64 blocks), after the caller's argument checks.
static int prepare_streaming(int x_dtype, const StreamSegs& segs, int64_t M, int64_t K,
                             int64_t n_cols, int gs, int bits, const dfmi_qmm_tuning* tuning,
                             void* workspace, size_t workspace_bytes, StreamLaunch& L) {
  StreamPlan& p = L.p;
  int64_t Ns[kMaxSeg];
  for (int i = 0; i < segs.nseg; ++i) Ns[i] = segs.seg[i].N;
  const int rc = plan_stream(M, K, n_cols, gs, bits, tuning, p, Ns, segs.nseg);
  if (rc != DFMI_OK) return rc;
  // a fused pair table only where the fused kernel takes the plan (else the
  // segments' own tables, or none: the window kernel, the same sums)
  if (M > 63 || p.kp >= 512 || p.chunks >= 65536) {  // the kernels' packed argument fields
    set_error("dfmi_qmm: plan outside the kernel's argument fields (M %lld, kp %d, steps %d)",
              (long long)M, p.kp, p.chunks);
    return DFMI_EINVAL;
  }
  StreamSegs sg = segs;
  if (sg.fused && !(p.tsb && fused_fits(sg, p.whole, p.kp, p.chunks, (int)M))) sg.fused = nullptr;
  if (p.rw == 2 && !segs_have_pairs(sg)) plan_as_rows64(p);
  // each matrix's first block in the launch's block size
  StreamSegs& m = L.m;
  m = sg;
  int blk = 0;
  for (int i = 0; i < m.nseg; ++i) {
    m.seg[i].blk0 = blk;
    blk += (int)((Ns[i] + kStreamRows * p.rw - 1) / (kStreamRows * p.rw));
  }
  StreamArgs& a = L.a;
  a.x = nullptr;
  a.partials = nullptr;
  a.counters = nullptr;
  if (p.kp > 1) {
    if (!workspace || workspace_bytes < p.ws_bytes || !aligned16(workspace)) {
      set_error("dfmi_qmm: workspace of %zu bytes (16-byte aligned) required, got %zu",
                p.ws_bytes, workspace_bytes);
      return DFMI_ENOSPC;
    }
    a.counters = static_cast<uint32_t*>(workspace);
    a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  a.M = (int)M;
  a.K = (int)K;
  a.chunks = p.chunks;
  a.kp = p.kp;
  a.n_blocks = p.n_blocks;
  a.xcd_map = p.xcd_map;
  a.pstride = kStreamRows * p.rw * (p.n_blocks - p.whole);
  a.whole = p.whole;
  L.x_dtype = x_dtype;
  L.gs = gs;
  allow_lds_all();
  return DFMI_OK;
}

// Launch a prepared streaming plan on x (the outputs are in L.m).
static int run_streaming(const StreamLaunch& L, const void* x, hipStream_t st) {
  StreamArgs a = L.a;
  a.x = static_cast<const uint16_t*>(x);
  if (L.x_dtype == DFMI_BF16) launch_stream<BF16>(L.gs, L.p, st, a, L.m);
  else launch_stream<F16>(L.gs, L.p, st, a, L.m);
  return check_launch(L.m.nseg == 1 ? "dfmi_qmm_affine" : "dfmi_qmm_affine_multi");
}

// The streaming kernel over the matrices of segs, after the caller's
// argument checks.
static int launch_streaming(const void* x, int x_dtype, const StreamSegs& segs, int64_t M,
                            int64_t K, int64_t n_cols, int gs, int bits,
                            const dfmi_qmm_tuning* tuning, void* workspace,
                            size_t workspace_bytes, hipStream_t st) {
  StreamLaunch L;
  const int rc = prepare_streaming(x_dtype, segs, M, K, n_cols, gs, bits, tuning, workspace,
                                   workspace_bytes, L);
  if (rc != DFMI_OK) return rc;
  return run_streaming(L, x, st);
}

// Shared-activation launches take the streaming kernel when every matrix
// does (their blocks then form one grid); the columns of that grid, 64 per
// block, or 0.
static int64_t multi_stream_cols(int64_t M, int64_t K, const int64_t* Ns, int nseg, int gs,
                                 int bits) {
  int64_t blocks = 0;
  for (int i = 0; i < nseg; ++i) {
    if (!use_stream(M, K, Ns[i], gs, bits, nullptr)) return 0;
    blocks += (Ns[i] + kStreamRows - 1) / kStreamRows;
  }
  if (blocks > kMaxCounters && K / gs > sb_max_groups(bits == 8 ? 8 : kSbPieces)) return 0;
  if (blocks * kStreamRows >= (1ll << 31) / 32) return 0;
  return blocks * kStreamRows;
}

extern "C" size_t dfmi_qmm_workspace_bytes_ex(int64_t M, int64_t K, int64_t N, int group_size,
                                              int bits, const dfmi_qmm_tuning* tuning) {
  if (validate_qmm(DFMI_BF16, M, K, N, group_size, bits) != DFMI_OK || M == 0 || N == 0 ||
      !valid_path(tuning))
    return 0;
  if (!use_stream(M, K, N, group_size, bits, tuning)) return 0;
  StreamPlan p;
  if (plan_stream(M, K, N, group_size, bits, tuning, p) != DFMI_OK) return 0;
  return p.ws_bytes;
}

extern "C" int dfmi_qmm_plan(int64_t M, int64_t K, const int64_t* Ns, int nseg, int group_size,
                             int bits, const dfmi_qmm_tuning* tuning, dfmi_qmm_plan_info* out) {
  if (!Ns || !out || nseg < 1 || nseg > kMaxSeg || !valid_path(tuning) ||
      (nseg > 1 && tuning)) {
    set_error("dfmi_qmm_plan: bad arguments");
    return DFMI_EINVAL;
  }
  for (int i = 0; i < nseg; ++i) {
    const int rc = validate_qmm(DFMI_BF16, M, K, Ns[i], group_size, bits);
    if (rc != DFMI_OK) return rc;
  }
  *out = dfmi_qmm_plan_info{};
  int64_t cols = 0;
  if (nseg == 1) {
    if (!use_stream(M, K, Ns[0], group_size, bits, tuning))
      return DFMI_OK;  // not the streaming kernel: streaming = 0
    cols = Ns[0];
  } else {
    cols = multi_stream_cols(M, K, Ns, nseg, group_size, bits);
    if (cols <= 0) return DFMI_OK;
  }
  StreamPlan p;
  const int rc = plan_stream(M, K, cols, group_size, bits, tuning, p, Ns, nseg);
  if (rc != DFMI_OK) return rc;
  out->streaming = 1;
  out->rows_per_block = kStreamRows * p.rw;
  out->waves = p.WV;
  out->k_splits = p.kp;
  out->whole_blocks = p.whole;
  out->blocks = p.n_blocks;
  out->workgroups = p.grid_x;
  out->pair_streaming = p.tsb;
  return DFMI_OK;
}

extern "C" const char* dfmi_qmm_kernel_name(int64_t M, int64_t K, int64_t N, int group_size,
                                             int bits, const dfmi_qmm_tuning* tuning) {
  if (validate_qmm(DFMI_BF16, M, K, N, group_size, bits) != DFMI_OK || !valid_path(tuning))
    return nullptr;
  if (bits == 8) return use_stream(M, K, N, group_size, bits, tuning) ? "qmm8_stream_kernel"
                                                                      : "qmm8_kernel";
  return use_stream(M, K, N, group_size, bits, tuning) ? "qmm_stream_kernel" : "qmm_dense_kernel";
}

extern "C" size_t dfmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size,
                                           int bits) {
  return dfmi_qmm_workspace_bytes_ex(M, K, N, group_size, bits, nullptr);
}

extern "C" int dfmi_qmm_affine_pairs(const void* x, int x_dtype, const uint32_t* w_q,
                                     const void* scales, const void* biases,
                                     const uint32_t* sb_pairs, void* y, int64_t M, int64_t K,
                                     int64_t N, int group_size, int bits, void* workspace,
                                     size_t workspace_bytes, const dfmi_qmm_tuning* tuning,
                                     void* stream) {
  int rc = validate_qmm(x_dtype, M, K, N, group_size, bits);
  if (rc != DFMI_OK) return rc;
  if (!valid_path(tuning)) {
    set_error("dfmi_qmm: tuning path %d unsupported (0 auto, 1 general, 2 streaming)",
              tuning->path);
    return DFMI_EINVAL;
  }
  if (M == 0 || N == 0) return DFMI_OK;
  // a forced streaming plan on a shape outside the streaming kernel is an
  // error for both weight widths (checked before the 8-bit fallback)
  if (tuning && tuning->path == 2 && !use_stream(M, K, N, group_size, bits, tuning)) {
    set_error("dfmi_qmm: shape M=%lld K=%lld N=%lld gs=%d bits=%d outside the streaming kernel",
              (long long)M, (long long)K, (long long)N, group_size, bits);
    return DFMI_EINVAL;
  }
  if (!x || !w_q || !scales || !biases || !y) {
    set_error("dfmi_qmm: null pointer");
    return DFMI_EINVAL;
  }
  if (!aligned16(x) || !aligned16(w_q) || !aligned16(scales) || !aligned16(biases) ||
      (sb_pairs && !aligned16(sb_pairs))) {
    set_error("dfmi_qmm: x, w_q, scales, biases and sb_pairs must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  // 8-bit: the streaming kernel where it applies, else the register-load kernel
  if (bits == 8 && !use_stream(M, K, N, group_size, bits, tuning))
    return dfmi_qmm8_launch(x, x_dtype, w_q, scales, biases, y, M, K, N, group_size, stream);
  if (use_stream(M, K, N, group_size, bits, tuning)) {
    StreamSegs m{};
    m.seg[0] = StreamSeg{w_q, static_cast<const uint16_t*>(scales),
                         static_cast<const uint16_t*>(biases), static_cast<uint16_t*>(y), (int)N, 0,
                         sb_pairs};
    m.nseg = 1;
    return launch_streaming(x, x_dtype, m, M, K, N, group_size, bits, tuning, workspace,
                            workspace_bytes, st);
  }
  DensePlan p;
  rc = plan_dense(M, K, N, tuning, p);
  if (rc != DFMI_OK) return rc;
  DenseArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = w_q;
  a.s = static_cast<const uint16_t*>(scales);
  a.b = static_cast<const uint16_t*>(biases);
  a.y = static_cast<uint16_t*>(y);
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.chunks = p.chunks;
  if (x_dtype == DFMI_BF16) launch_tag<BF16>(group_size, p, st, a);
  else launch_tag<F16>(group_size, p, st, a);
  return check_launch("dfmi_qmm_affine");
}

extern "C" int dfmi_qmm_affine_ex(const void* x, int x_dtype, const uint32_t* w_q,
                                  const void* scales, const void* biases, void* y, int64_t M,
                                  int64_t K, int64_t N, int group_size, int bits, void* workspace,
                                  size_t workspace_bytes, const dfmi_qmm_tuning* tuning,
                                  void* stream) {
  return dfmi_qmm_affine_pairs(x, x_dtype, w_q, scales, biases, nullptr, y, M, K, N, group_size,
                               bits, workspace, workspace_bytes, tuning, stream);
}

extern "C" int dfmi_qmm_affine(const void* x, int x_dtype, const uint32_t* w_q, const void* scales,
                               const void* biases, void* y, int64_t M, int64_t K, int64_t N,
                               int group_size, int bits, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return dfmi_qmm_affine_ex(x, x_dtype, w_q, scales, biases, y, M, K, N, group_size, bits,
                            workspace, workspace_bytes, nullptr, stream);
}

// ---------------------------------------------------------------------------
// dfmi_qmm_affine_noalloc: dfmi_qmm_affine with its split-K workspace (block
// counters, then fp32 partials) in this static device array instead of a
// caller's buffer, for callers that cannot allocate device memory.  Each GPU
// the library runs on holds one copy until the process ends.  In host code
// `scratch` names a host-side stand-in; the device address of each GPU's copy
// comes from hipGetSymbolAddress, once per device, and only that address is
// passed to kernels.
constexpr size_t kScratchBytes = kCounterBytes + ((size_t)8 << 20);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace dfmi {

constexpr int kScratchDevices = 64;

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

// This device's copy of `scratch`.  Until a call on the device has run
// outside graph capture, each call first clears the counter region with a
// kernel on `st` (ahead of the caller's launch in stream order).  A call
// under capture records that clear into the graph, so every replay starts
// from zero counters, and does not count as the device's first call: the
// graph may never be replayed, so the next uncaptured call clears again.
static int scratch_of_device(hipStream_t st, void** out) {
  static std::mutex mu;
  static void* ptrs[kScratchDevices] = {};
  static bool cleared[kScratchDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_error("dfmi_qmm_affine_noalloc: no usable current device (%s, device %d)",
              hipGetErrorString(e), dev);
    return DFMI_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("dfmi_qmm_affine_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(e));
      return DFMI_ELAUNCH;
    }
    ptrs[dev] = p;
  }
  if (!cleared[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cap);
    if (e != hipSuccess) {
      set_error("dfmi_qmm_affine_noalloc: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
      return DFMI_ELAUNCH;
    }
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, st,
                       static_cast<uint32_t*>(ptrs[dev]), (int)(kCounterBytes / 4));
    const int rc = check_launch("dfmi_qmm_affine_noalloc (scratch clear)");
    if (rc != DFMI_OK) return rc;
    if (cap == hipStreamCaptureStatusNone) cleared[dev] = true;
  }
  *out = ptrs[dev];
  return DFMI_OK;
}

}  // namespace dfmi

extern "C" size_t dfmi_qmm_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int dfmi_qmm_affine_noalloc(const void* x, int x_dtype, const uint32_t* w_q,
                                       const void* scales, const void* biases, void* y, int64_t M,
                                       int64_t K, int64_t N, int group_size, int bits,
                                       void* stream) {
  int rc = validate_qmm(x_dtype, M, K, N, group_size, bits);
  if (rc != DFMI_OK) return rc;
  if (M == 0 || N == 0) return DFMI_OK;
  const size_t need = dfmi_qmm_workspace_bytes_ex(M, K, N, group_size, bits, nullptr);
  if (need > kScratchBytes) {
    set_error("dfmi_qmm_affine_noalloc: shape M=%lld K=%lld N=%lld needs %zu workspace bytes, "
              "above the %zu-byte static scratch (use dfmi_qmm_affine with a workspace)",
              (long long)M, (long long)K, (long long)N, need, kScratchBytes);
    return DFMI_ENOSPC;
  }
  void* ws = nullptr;
  rc = scratch_of_device(static_cast<hipStream_t>(stream), &ws);
  if (rc != DFMI_OK) return rc;
  return dfmi_qmm_affine_ex(x, x_dtype, w_q, scales, biases, y, M, K, N, group_size, bits, ws,
                            kScratchBytes, nullptr, stream);
}

extern "C" size_t dfmi_qmm_multi_workspace_bytes(int64_t M, int64_t K, const int64_t* Ns,
                                                 int nseg, int group_size, int bits) {
  if (!Ns || nseg < 1 || nseg > kMaxSeg) return 0;
  for (int i = 0; i < nseg; ++i)
    if (validate_qmm(DFMI_BF16, M, K, Ns[i], group_size, bits) != DFMI_OK) return 0;
  if (M == 0) return 0;
  const int64_t cols = multi_stream_cols(M, K, Ns, nseg, group_size, bits);
  if (cols > 0) {
    StreamPlan p;
    return plan_stream(M, K, cols, group_size, bits, nullptr, p, Ns, nseg) == DFMI_OK ? p.ws_bytes
                                                                                   : 0;
  }
  size_t ws = 0;
  for (int i = 0; i < nseg; ++i)
    ws = std::max(ws, dfmi_qmm_workspace_bytes_ex(M, K, Ns[i], group_size, bits, nullptr));
  return ws;
}

extern "C" const char* dfmi_qmm_multi_kernel_name(int64_t M, int64_t K, const int64_t* Ns,
                                                   int nseg, int group_size, int bits) {
  if (!Ns || nseg < 1 || nseg > kMaxSeg) return nullptr;
  for (int i = 0; i < nseg; ++i)
    if (validate_qmm(DFMI_BF16, M, K, Ns[i], group_size, bits) != DFMI_OK) return nullptr;
  if (multi_stream_cols(M, K, Ns, nseg, group_size, bits) <= 0) return nullptr;
  return nseg == 1 ? "qmm_stream_kernel" : "qmm_stream_multi_kernel";
}

// dfmi_qmm_affine_multi / _multi_fused; fused: the matrices' pair tables side
// by side ([K/gs][sum of N]), or null.
static int qmm_multi(const void* x, int x_dtype, const dfmi_qmm_segment* segs, int nseg,
                     const uint32_t* fused, int64_t M, int64_t K, int group_size, int bits,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!segs || nseg < 1 || nseg > kMaxSeg) {
    set_error("dfmi_qmm_multi: 1..%d segments required (got %d)", kMaxSeg, nseg);
    return DFMI_EINVAL;
  }
  int64_t Ns[kMaxSeg];
  for (int i = 0; i < nseg; ++i) {
    const int rc = validate_qmm(x_dtype, M, K, segs[i].N, group_size, bits);
    if (rc != DFMI_OK) return rc;
    Ns[i] = segs[i].N;
  }
  if (M == 0) return DFMI_OK;
  if (!x || !aligned16(x)) {
    set_error("dfmi_qmm_multi: x must be a 16-byte aligned device pointer");
    return DFMI_EINVAL;
  }
  for (int i = 0; i < nseg; ++i) {
    if (segs[i].N == 0) continue;  // nothing of an empty matrix is read or written
    if (!segs[i].w_q || !segs[i].scales || !segs[i].biases || !segs[i].y) {
      set_error("dfmi_qmm_multi: null pointer in segment %d", i);
      return DFMI_EINVAL;
    }
    if (!aligned16(segs[i].w_q) || !aligned16(segs[i].scales) || !aligned16(segs[i].biases) ||
        (segs[i].sb_pairs && !aligned16(segs[i].sb_pairs))) {
      set_error("dfmi_qmm_multi: segment %d: w_q, scales, biases and sb_pairs must be 16-byte "
                "aligned", i);
      return DFMI_EINVAL;
    }
  }
  const int64_t cols = multi_stream_cols(M, K, Ns, nseg, group_size, bits);
  if (cols > 0) {
    StreamSegs m{};
    int blk = 0;
    for (int i = 0; i < nseg; ++i) {
      m.seg[i] = StreamSeg{segs[i].w_q, static_cast<const uint16_t*>(segs[i].scales),
                           static_cast<const uint16_t*>(segs[i].biases),
                           static_cast<uint16_t*>(segs[i].y), (int)Ns[i], blk, segs[i].sb_pairs};
      blk += (int)((Ns[i] + kStreamRows - 1) / kStreamRows);
    }
    m.nseg = nseg;
    m.fused = fused;
    return launch_streaming(x, x_dtype, m, M, K, cols, group_size, bits, nullptr, workspace,
                            workspace_bytes, static_cast<hipStream_t>(stream));
  }
  // one launch per matrix, in order on the stream (they may share the workspace)
  for (int i = 0; i < nseg; ++i) {
    const int rc = dfmi_qmm_affine_pairs(x, x_dtype, segs[i].w_q, segs[i].scales,
                                         segs[i].biases, segs[i].sb_pairs, segs[i].y, M, K,
                                         segs[i].N, group_size, bits, workspace, workspace_bytes,
                                         nullptr, stream);
    if (rc != DFMI_OK) return rc;
  }
  return DFMI_OK;
}

extern "C" int dfmi_qmm_affine_multi(const void* x, int x_dtype, const dfmi_qmm_segment* segs,
                                     int nseg, int64_t M, int64_t K, int group_size, int bits,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  return qmm_multi(x, x_dtype, segs, nseg, nullptr, M, K, group_size, bits, workspace,
                   workspace_bytes, stream);
}

extern "C" int dfmi_qmm_affine_multi_fused(const void* x, int x_dtype,
                                           const dfmi_qmm_segment* segs, int nseg,
                                           const uint32_t* sb_pairs, int64_t M, int64_t K,
                                           int group_size, int bits, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  if (sb_pairs && !aligned16(sb_pairs)) {
    set_error("dfmi_qmm_multi_fused: sb_pairs must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  return qmm_multi(x, x_dtype, segs, nseg, sb_pairs, M, K, group_size, bits, workspace,
                   workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Prepared launches (dfmi_qmm_prepare / dfmi_qmm_run): the plan, the kernel
// arguments and the matrices of a verify linear (or of sibling projections
// sharing their input) computed once, so that each call is one short C call.

namespace dfmi {

constexpr uint64_t kRecordMagic = 0x6466'6d69'7265'6301ull;  // "dfmirec", version 1

struct QmmRecord {
  uint64_t magic;
  int kind;  // 1: streaming launch (L); 2: dfmi_qmm_affine_multi_fused call with the stored arguments
  int nseg;
  StreamLaunch L;
  // kind 2
  dfmi_qmm_segment segs[kMaxSeg];
  const uint32_t* fused;
  int x_dtype, gs, bits;
  int64_t M, K;
  void* workspace;
  size_t workspace_bytes;
};
static_assert(sizeof(QmmRecord) <= DFMI_QMM_RECORD_BYTES, "record buffer");
static_assert(alignof(QmmRecord) <= 16, "record alignment");

}  // namespace dfmi

extern "C" int dfmi_qmm_prepare(int x_dtype, const dfmi_qmm_segment* segs, int nseg,
                                const uint32_t* fused_pairs, int64_t sb_stride, int64_t M,
                                int64_t K, int group_size, int bits, void* workspace,
                                size_t workspace_bytes, void* record, size_t record_bytes) {
  if (!record || record_bytes < sizeof(QmmRecord) ||
      (reinterpret_cast<uintptr_t>(record) & 15u)) {
    set_error("dfmi_qmm_prepare: record buffer of %zu bytes (16-byte aligned) required",
              sizeof(QmmRecord));
    return DFMI_EINVAL;
  }
  QmmRecord* r = static_cast<QmmRecord*>(record);
  r->magic = 0;  // invalid until prepared
  if (!segs || nseg < 1 || nseg > kMaxSeg) {
    set_error("dfmi_qmm_prepare: 1..%d segments required (got %d)", kMaxSeg, nseg);
    return DFMI_EINVAL;
  }
  int64_t Ns[kMaxSeg];
  for (int i = 0; i < nseg; ++i) {
    const int rc = validate_qmm(x_dtype, M, K, segs[i].N, group_size, bits);
    if (rc != DFMI_OK) return rc;
    Ns[i] = segs[i].N;
    if (segs[i].N == 0) continue;
    if (!segs[i].w_q || !segs[i].scales || !segs[i].biases) {
      set_error("dfmi_qmm_prepare: null pointer in segment %d", i);
      return DFMI_EINVAL;
    }
    if (!aligned16(segs[i].w_q) || !aligned16(segs[i].scales) || !aligned16(segs[i].biases) ||
        (segs[i].sb_pairs && !aligned16(segs[i].sb_pairs))) {
      set_error("dfmi_qmm_prepare: segment %d: w_q, scales, biases and sb_pairs must be 16-byte "
                "aligned", i);
      return DFMI_EINVAL;
    }
  }
  if (fused_pairs && !aligned16(fused_pairs)) {
    set_error("dfmi_qmm_prepare: fused_pairs must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  if (sb_stride != 0) {
    bool ok = !fused_pairs && sb_stride % 4 == 0 && sb_stride < (1ll << 31) &&
              sb_stride * (K / group_size) * 4 <= 0xFFFFFFFFll;
    // (N % 4 == 0: a lane's 16-byte load of four pairs then ends inside its
    // slice, so nothing past the wider table is read)
    for (int i = 0; i < nseg; ++i)
      ok = ok && (Ns[i] == 0 || (segs[i].sb_pairs && Ns[i] <= sb_stride && Ns[i] % 4 == 0));
    if (!ok) {
      set_error("dfmi_qmm_prepare: sb_stride %lld needs every matrix's pair table, "
                "N <= sb_stride, N %% 4 == 0, sb_stride %% 4 == 0 and no fused_pairs",
                (long long)sb_stride);
      return DFMI_EINVAL;
    }
  }
  const int64_t cols = nseg == 1 ? (use_stream(M, K, Ns[0], group_size, bits, nullptr) ? Ns[0] : 0)
                                 : multi_stream_cols(M, K, Ns, nseg, group_size, bits);
  if (M > 0 && cols > 0) {
    StreamSegs m{};
    int blk = 0;
    for (int i = 0; i < nseg; ++i) {
      m.seg[i] = StreamSeg{segs[i].w_q, static_cast<const uint16_t*>(segs[i].scales),
                           static_cast<const uint16_t*>(segs[i].biases), nullptr, (int)Ns[i], blk,
                           segs[i].sb_pairs};
      blk += (int)((Ns[i] + kStreamRows - 1) / kStreamRows);
    }
    m.nseg = nseg;
    m.fused = nseg > 1 ? fused_pairs : nullptr;
    m.tn = (uint32_t)sb_stride;
    const int rc = prepare_streaming(x_dtype, m, M, K, cols, group_size, bits, nullptr,
                                     workspace, workspace_bytes, r->L);
    if (rc != DFMI_OK) return rc;
    r->kind = 1;
  } else {
    // outside the streaming kernel: the shared-activation entry point's own
    // route at each call (a pair table in a wider one is not passed: the
    // plans it would serve are all streaming)
    for (int i = 0; i < nseg; ++i) {
      r->segs[i] = segs[i];
      r->segs[i].y = nullptr;
      if (sb_stride != 0) r->segs[i].sb_pairs = nullptr;
    }
    r->fused = fused_pairs;
    r->kind = 2;
  }
  r->nseg = nseg;
  r->x_dtype = x_dtype;
  r->gs = group_size;
  r->bits = bits;
  r->M = M;
  r->K = K;
  r->workspace = workspace;
  r->workspace_bytes = workspace_bytes;
  r->magic = kRecordMagic;
  return DFMI_OK;
}

extern "C" int dfmi_qmm_run(const void* record, const void* x, void* y0, void* y1, void* y2,
                            void* y3, void* stream) {
  const QmmRecord* r = static_cast<const QmmRecord*>(record);
  if (!r || r->magic != kRecordMagic) {
    set_error("dfmi_qmm_run: not a prepared record");
    return DFMI_EINVAL;
  }
  if (r->M == 0) return DFMI_OK;
  if (!x || !aligned16(x)) {
    set_error("dfmi_qmm_run: x must be a 16-byte aligned device pointer");
    return DFMI_EINVAL;
  }
  void* const ys[kMaxSeg] = {y0, y1, y2, y3};
  if (r->kind == 1) {
    StreamLaunch L = r->L;
    for (int i = 0; i < r->nseg; ++i) {
      if (L.m.seg[i].N > 0 && !ys[i]) {
        set_error("dfmi_qmm_run: null output %d", i);
        return DFMI_EINVAL;
      }
      L.m.seg[i].y = static_cast<uint16_t*>(ys[i]);
    }
    return run_streaming(L, x, static_cast<hipStream_t>(stream));
  }
  dfmi_qmm_segment segs[kMaxSeg];
  for (int i = 0; i < r->nseg; ++i) {
    segs[i] = r->segs[i];
    segs[i].y = ys[i];
  }
  return qmm_multi(x, r->x_dtype, segs, r->nseg, r->fused, r->M, r->K, r->gs, r->bits,
                   r->workspace, r->workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Pair table of the pair-streaming kernels: pairs[g][n] = scales[n][g] |
// biases[n][g] << 16 (16-bit values of either activation dtype).  Each
// workgroup transposes a 64 (rows) x 64 (groups) tile through LDS so that
// both the reads (along groups) and the writes (along rows) are contiguous.
__global__ __launch_bounds__(256) void sb_pairs_kernel(const uint16_t* s, const uint16_t* b,
                                                       uint32_t* t, int N, int G) {
  __shared__ uint32_t tile[64][65];
  const int n0 = blockIdx.x * 64, g0 = blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, c = i % 64;  // row n0 + r, group g0 + c
    const int n = n0 + r, g = g0 + c;
    uint32_t v = 0;
    if (n < N && g < G) {
      const int64_t o = (int64_t)n * G + g;
      v = (uint32_t)s[o] | ((uint32_t)b[o] << 16);
    }
    tile[r][c] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int c = i / 64, r = i % 64;  // group g0 + c, row n0 + r
    const int n = n0 + r, g = g0 + c;
    if (n < N && g < G) t[(int64_t)g * N + n] = tile[r][c];
  }
}

extern "C" int dfmi_sb_pairs(const void* scales, const void* biases, int dtype, int64_t N,
                             int64_t groups, uint32_t* sb_pairs, void* stream) {
  if (dtype != DFMI_BF16 && dtype != DFMI_F16) {
    set_error("dfmi_sb_pairs: dtype %d unsupported (bf16 or f16)", dtype);
    return DFMI_EINVAL;
  }
  if (N < 0 || groups < 0 || N >= (1ll << 31) || groups >= (1ll << 31) ||
      N * groups * 4 > 0xFFFFFFFFll) {
    set_error("dfmi_sb_pairs: bad shape N=%lld groups=%lld", (long long)N, (long long)groups);
    return DFMI_EINVAL;
  }
  if (N == 0 || groups == 0) return DFMI_OK;
  if (!scales || !biases || !sb_pairs) {
    set_error("dfmi_sb_pairs: null pointer");
    return DFMI_EINVAL;
  }
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((groups + 63) / 64));
  hipLaunchKernelGGL(sb_pairs_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases),
                     sb_pairs, (int)N, (int)groups);
  return check_launch("dfmi_sb_pairs");
}
