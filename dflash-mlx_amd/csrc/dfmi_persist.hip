// Persistent streaming matmul: y_i[M, N_i] = x[M, K] . dequant(W_i)^T for
// up to three weight matrices W_i that share the activations x (one matrix
// for a plain verify linear; the q/k/v or gate/up siblings of a layer in one
// launch).  M <= 16, int4, K % 256 == 0.
//
// Work is cut into units of 64 weight rows (one block of one matrix) over a
// K range.  Workgroups of 4 wavefronts, two per CU (80 KB of LDS each: two
// independent barriers per CU, so one workgroup's waits are the other's
// compute), each stream a list of units through ONE pipeline: the Stream
// main loop (three LDS stages, activation + weight DMA per 256-k step,
// fragments of the next step read while the current one computes) runs
// across unit boundaries, so a unit's first steps are fetched while the
// previous unit computes and no workgroup pays more than one pipeline fill.
// The scale / bias window is one buffer: the next unit's window is fetched
// as soon as every wavefront has read the last step of the current one.
//
// Work partition (stream-K): the U blocks x S steps of the launch form one
// sequence of T = U S block-steps; workgroup w takes the contiguous range
// [w T / G, (w + 1) T / G).  Blocks wholly inside a range are whole units
// (stored directly); a range starts and ends with at most one partial block
// each.  A partial block's fp32 tile goes to the workspace (slot 0 for the
// workgroup's first unit, slot 1 for its last) without waiting; at its end
// the workgroup waits for its own writes and bumps the counters of its
// partial blocks; the last workgroup to arrive at a block sums that block's
// parts in workgroup order (deterministic) and writes y.  Nothing is in
// flight at that point, so the exchange never drains the pipeline.
//
// Memory ordering.  The workgroups of a block run on different XCDs, whose
// L2 caches are not coherent with each other within a launch, and a plain
// load of a partial can return a line an XCD cached in an earlier launch.
// So partial tiles are written and read with agent-scope atomic RMWs
// (swap; or with 0), which are performed at the same coherence point as the
// counters' RMWs: a writer's RMWs have completed (vmcnt 0) before its counter
// increment is issued, and the last arriver issues its reads after its own
// increment returned the final count.
//
// Per-unit epilogue: the 4 wavefronts' partial tiles are summed through the
// LDS stage whose fragments were read last (its next DMA comes only after
// the next wait's barrier), then stored.
//
// Wait accounting: every wavefront issues the same DMA instructions per step
// (Stream::CHUNK_DMA) and per window (Stream::SB_DMA), so the number of loads
// issued after any step is known exactly; a wait lets those stay in flight.
// Epilogue stores are left out of the count: a store can only lengthen a
// wait (a pending load keeps every younger load pending too).
#include <algorithm>

#include "dfmi_host.h"
#include "dfmi_stream.h"

namespace dfmi {

constexpr int kPMaxSeg = 3;
constexpr int kPStages = 3;
constexpr int kPWaves = 4;
constexpr int kPGroups = 512;            // workgroups: two per CU
constexpr size_t kPCounterBytes = 65536;  // one counter per block
constexpr int kPMaxBlocks = (int)(kPCounterBytes / 4);

struct PSeg {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int N;     // rows of this matrix
  int blk0;  // first global block of this matrix
};

struct PArgs {
  const uint16_t* x;
  PSeg seg[kPMaxSeg];
  float* partials;     // partial blocks: [workgroup][2][16][64] fp32
  uint32_t* counters;  // [block], zero between calls
  int M, K;
  int S;  // 256-k steps of K
  int T;  // block-steps of the launch (U S)
  int G;  // workgroups
};

template <typename Tag, int GS>
struct PLayout {
  using S = Stream<Tag, GS, 1, kPWaves, kSbPieces, 4>;
  static_assert(S::DEPTH == kPStages, "stages");
  static constexpr int BYTES = S::LDS_BYTES;
  static_assert(BYTES <= 80 * 1024, "two workgroups per CU");
  static_assert(S::XBUF == 2 * S::RED_FLOATS * 4 && S::WBUF == 2 * S::RED_FLOATS * 4,
                "epilogue: two wavefronts' partial tiles per activation or weight stage");
};

// LDS reads and writes done, then the workgroup barrier; loads stay in flight.
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // vmcnt 63, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename Tag, int GS, int NSEG>
__global__ __launch_bounds__(64 * kPWaves) void qmm_persist_kernel(PArgs a) {
  using LY = PLayout<Tag, GS>;
  using S = typename LY::S;
  constexpr int NT = 64 * kPWaves;
  constexpr int PER = S::RED_FLOATS / NT;  // outputs per thread of a unit (64 x 16 / 256)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = blockIdx.x;
  const int K = a.K, M = a.M, Sfull = a.S, T = a.T, G = a.G;
  // this workgroup's block-steps [t0, t1): blocks u0 .. u0 + nunits - 1
  const int t0 = (int)((int64_t)g * T / G), t1 = (int)((int64_t)(g + 1) * T / G);
  const int V = t1 - t0;  // positions (unit, step)
  if (V <= 0) return;     // uniform
  const int u0 = t0 / Sfull;
  const int nunits = (t1 - 1) / Sfull - u0 + 1;
  const int first_c0 = t0 - u0 * Sfull;
  const int last_c1 = t1 - (u0 + nunits - 1) * Sfull;

  // the arguments as plain values (lambdas capture these, never the struct)
  // (entries past NSEG repeat entry 0: never selected, never loaded)
  const uint32_t* sw[kPMaxSeg];
  const uint16_t* ss[kPMaxSeg];
  const uint16_t* sbi[kPMaxSeg];
  uint16_t* sy[kPMaxSeg];
  int sN[kPMaxSeg], sblk[kPMaxSeg];
#pragma unroll
  for (int i = 0; i < kPMaxSeg; ++i) {
    const int k = i < NSEG ? i : 0;
    sw[i] = a.seg[k].w;
    ss[i] = a.seg[k].s;
    sbi[i] = a.seg[k].b;
    sy[i] = a.seg[k].y;
    sN[i] = a.seg[k].N;
    sblk[i] = a.seg[k].blk0;
  }
  const uint16_t* const ax = a.x;
  float* const apart = a.partials;
  uint32_t* const acnt = a.counters;
  const int groups = K / GS;

  auto unit_block = [&](int j) { return u0 + j; };
  auto seg_of = [&](int u) {
    int si = 0;
#pragma unroll
    for (int i = 1; i < NSEG; ++i) si += (int)(u >= sblk[i]);
    return si;
  };
#define DFMI_PSEL(arr, i) \
  (NSEG == 1 ? arr[0] : ((i) == 0 ? arr[0] : (i) == 1 ? arr[1] : arr[2]))
  auto unit_c0 = [&](int j) { return j == 0 ? first_c0 : 0; };
  auto unit_c1 = [&](int j) { return j == nunits - 1 ? last_c1 : Sfull; };
  // a unit other workgroups also work on
  auto is_part = [&](int j) { return unit_c0(j) != 0 || unit_c1(j) != Sfull; };
  // the workgroup whose range holds block-step t
  auto owner = [&](int t) { return (int)(((int64_t)(t + 1) * G - 1) / T); };

  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(ax, (uint32_t)M * (uint32_t)K * 2u);
  const DqConst dq = dq_const<Tag>();
  typename S::Lane L;
  {
    typename S::Ctx c0x;
    c0x.x = xr;
    c0x.dense();
    c0x.K = K;
    c0x.M = M;
    c0x.N = 1;
    c0x.groups = groups;
    c0x.n0 = 0;
    c0x.lane = lane;
    c0x.wave = wave;
    L = S::lane_setup(c0x);
  }
  // unit j's context for the DMA: its matrix's buffers and first row
  auto unit_ctx = [&](int j, typename S::Ctx& cx) __attribute__((always_inline)) {
    const int u = unit_block(j);
    const int si = seg_of(u);
    const int N = DFMI_PSEL(sN, si);
    cx.x = xr;
    cx.w = buffer_rsrc(DFMI_PSEL(sw, si), (uint32_t)N * (uint32_t)(K / 2));
    cx.s = buffer_rsrc(DFMI_PSEL(ss, si), (uint32_t)N * (uint32_t)groups * 2u);
    cx.b = buffer_rsrc(DFMI_PSEL(sbi, si), (uint32_t)N * (uint32_t)groups * 2u);
    cx.xrows = nullptr;
    cx.xbase = 0;
    cx.split = S::NB;
    cx.w2 = cx.w;
    cx.s2 = cx.s;
    cx.b2 = cx.b;
    cx.K = K;
    cx.M = M;
    cx.N = N;
    cx.groups = groups;
    cx.n0 = (u - DFMI_PSEL(sblk, si)) * S::NB;
    cx.lane = lane;
    cx.wave = wave;
    cx.sb_base = 0;
  };

  int ops = 0;  // DMA instructions this wavefront has issued
  // loads issued up to and including the chunks of positions q, q + 1, q + 2
  // after issue_next(q + 2) (oldest first), for the waits.  They move once per
  // position, also for positions past the range (no chunk: the mark is the
  // count so far), so a wait for position p + 1 always reads its own mark.
  int m0 = 0, m1 = 0, m2 = 0;
  // issue cursor: the next position to issue, as (unit, step)
  int ij = 0, ic = unit_c0(0);
  auto issue_window = [&](int j) __attribute__((always_inline)) {
    typename S::Ctx cx;
    unit_ctx(j, cx);
    const int piece0 = (unit_c0(j) * S::GPC) >> 3;
    S::issue_sb(cx, piece0, ((unit_c1(j) * S::GPC + 7) >> 3) - piece0);
    ops += S::SB_DMA;
  };
  // position p's chunk (p < V), then the marks move on by one position
  auto issue_next = [&](int p) __attribute__((always_inline)) {
    if (p < V) {
      typename S::Ctx cx;
      unit_ctx(ij, cx);
      if (ic == unit_c0(ij)) L = S::lane_setup(cx);  // a new unit's weight rows
      S::issue_chunk(cx, L, ic, __builtin_amdgcn_readfirstlane(p % kPStages));
      ops += S::CHUNK_DMA;
      if (++ic == unit_c1(ij)) {
        ++ij;
        ic = unit_c0(ij);
      }
    }
    m0 = m1;
    m1 = m2;
    m2 = ops;
  };
  // read cursor (the position whose fragments are read next)
  int rj = 0, rc = unit_c0(0);
  auto read_next = [&](int p, typename S::Frag& f) __attribute__((always_inline)) {
    typename S::Ctx cr;
    cr.wave = wave;
    cr.sb_base = 0;
    const int g0w = ((unit_c0(rj) * S::GPC) >> 3) * 8;
    S::read_frag(cr, L, rc, __builtin_amdgcn_readfirstlane(p % kPStages), g0w, f);
    if (++rc == unit_c1(rj)) {
      ++rj;
      rc = unit_c0(rj);
    }
  };

  f32x4 acc[S::NT][1];
  // unit j's outputs, summed through stage `slot`
  auto epilogue = [&](int j, int slot) __attribute__((always_inline)) {
    const int u = unit_block(j);
    const int si = seg_of(u);
    const int N = DFMI_PSEL(sN, si);
    uint16_t* y = DFMI_PSEL(sy, si);
    const int n0 = (u - DFMI_PSEL(sblk, si)) * S::NB;
    float* rx = reinterpret_cast<float*>(dfmi_smem + S::X_OFF + slot * S::XBUF);
    float* rw = reinterpret_cast<float*>(dfmi_smem + S::W_OFF + slot * S::WBUF);
    lds_barrier();  // every wavefront's fragment reads of that stage have returned
    {
      float* mine = (wave < 2 ? rx : rw) + (wave & 1) * S::RED_FLOATS;
#pragma unroll
      for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mine[(t * 4 + r) * 64 + lane] = acc[t][0][r];
    }
    lds_barrier();
    float v[PER];
    int mi[PER], ni[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int el = q * NT + tid;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kPWaves; ++w) sum += ((w < 2 ? rx : rw) + (w & 1) * S::RED_FLOATS)[el];
      v[q] = sum;
      const int l = el & 63, jj = (el >> 6) & 3, t = el >> 8;
      mi[q] = 4 * (l >> 4) + jj;
      ni[q] = 16 * t + (l & 15);  // row within the block
    }
    const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(y, (uint32_t)M * (uint32_t)N * 2u);
    if (!is_part(j)) {
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int n = n0 + ni[q];
        const uint32_t off =
            (mi[q] < M && n < N) ? (uint32_t)(mi[q] * N + n) * 2u : kNoRow;
        __builtin_amdgcn_raw_buffer_store_b16(Num<Tag>::f2h(v[q]), yr, off, 0, 0);
      }
      return;
    }
    // a partial block: its tile to this workgroup's slot, summed at the end
    // (atomic swaps: performed where the counters' atomics are, so no cache
    // of any XCD can hold a stale copy for the reader)
    uint32_t* part = reinterpret_cast<uint32_t*>(apart) + ((int64_t)g * 2 + (j == 0 ? 0 : 1)) * (16 * 64);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      // the returning form: its completion (vmcnt) means the swap was performed
      const uint32_t old = __hip_atomic_exchange(part + mi[q] * 64 + ni[q], __float_as_uint(v[q]),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("" ::"v"(old));
    }
  };
  // At the workgroup's end (nothing in flight): the exchange for a partial
  // block of unit j; the last workgroup to arrive sums the parts in
  // workgroup order and writes y.
  auto finish_part = [&](int j) __attribute__((always_inline)) {
    const int u = unit_block(j);
    const int si = seg_of(u);
    const int N = DFMI_PSEL(sN, si);
    uint16_t* y = DFMI_PSEL(sy, si);
    const int n0 = (u - DFMI_PSEL(sblk, si)) * S::NB;
    const int wf = owner(u * Sfull), wl = owner(u * Sfull + Sfull - 1);
    int* s_last = reinterpret_cast<int*>(dfmi_smem + S::X_OFF);
    stage_barrier<0>();  // every store of the workgroup has completed
    if (tid == 0) {
      const unsigned prev =
          __hip_atomic_fetch_add(&acnt[u], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = (prev == (unsigned)(wl - wf)) ? 1 : 0;
    }
    stage_barrier<0>();
    const bool last = *s_last != 0;
    stage_barrier<0>();  // s_last read by all before the next finish_part writes it
    if (!last) return;
    int mi[PER], ni[PER];
    float sum[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int el = q * NT + tid;
      const int l = el & 63, jj = (el >> 6) & 3;
      mi[q] = 4 * (l >> 4) + jj;
      ni[q] = 16 * (el >> 8) + (l & 15);
      sum[q] = 0.f;
    }
    for (int v0 = wf; v0 <= wl; v0 += 4) {
      // unconditional loads (a workgroup past wl re-reads wl's part and is
      // dropped), one memory round trip per four parts
      float t4[4][PER];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = min(v0 + i, wl);
        // block u is the first unit of workgroup v exactly when v's range
        // starts inside it
        const int slot = ((int)((int64_t)v * T / G) / Sfull == u) ? 0 : 1;
        uint32_t* src = reinterpret_cast<uint32_t*>(apart) + ((int64_t)v * 2 + slot) * (16 * 64);
#pragma unroll
        for (int q = 0; q < PER; ++q)
          t4[i][q] = __uint_as_float(__hip_atomic_fetch_or(src + mi[q] * 64 + ni[q], 0u,
                                                           __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < PER; ++q) sum[q] += (v0 + i <= wl) ? t4[i][q] : 0.f;
    }
    const __amdgpu_buffer_rsrc_t yr = buffer_rsrc(y, (uint32_t)M * (uint32_t)N * 2u);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int n = n0 + ni[q];
      const uint32_t off = (mi[q] < M && n < N) ? (uint32_t)(mi[q] * N + n) * 2u : kNoRow;
      __builtin_amdgcn_raw_buffer_store_b16(Num<Tag>::f2h(sum[q]), yr, off, 0, 0);
    }
    if (tid == 0)
      __hip_atomic_exchange(&acnt[u], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };

  issue_window(0);
  for (int k = 0; k < kPStages; ++k) issue_next(k);
  // position 0 landed: the window precedes it, the later chunks may be in flight
  stage_barrier_n(ops - m0);
  typename S::Frag fa, fb;
  read_next(0, fa);
  int cj = 0, cc = unit_c0(0);  // compute cursor
  // iteration p: position p + 1 must be in LDS (p + 2, p + 3 may be in
  // flight); position p's fragments are in CUR.  When p + 1 starts a new
  // unit, its window is fetched once every wavefront is past the last read
  // of the current window (the wait's barrier), and waited for before the
  // reads.
#define DFMI_PSTEP(p, CUR, NXT)                                                  \
  do {                                                                           \
    const bool last_ = cc == unit_c1(cj) - 1;                                    \
    if ((p) + 1 < V) {                                                           \
      stage_barrier_n(ops - m1); /* chunk p + 1 landed */                       \
      if (last_) issue_window(cj + 1);                                           \
      const int after_ = ops;                                                    \
      issue_next((p) + kPStages);                                                \
      if (last_) stage_barrier_n(ops - after_); /* the window landed */          \
      read_next((p) + 1, NXT);                                                   \
    }                                                                            \
    if (cc == unit_c0(cj)) {                                                     \
      _Pragma("unroll") for (int t = 0; t < S::NT; ++t) acc[t][0] = zero4();     \
    }                                                                            \
    S::compute(L, CUR, acc, dq);                                                 \
    if (last_) epilogue(cj, ((p) + 1) % kPStages);                               \
    if (++cc == unit_c1(cj)) {                                                   \
      ++cj;                                                                      \
      cc = unit_c0(cj);                                                          \
    }                                                                            \
  } while (0)
  int p = 0;
  for (; p + 1 < V; p += 2) {
    DFMI_PSTEP(p, fa, fb);
    DFMI_PSTEP(p + 1, fb, fa);
  }
  if (p < V) DFMI_PSTEP(p, fa, fb);
#undef DFMI_PSTEP
  if (is_part(0)) finish_part(0);
  if (nunits > 1 && is_part(nunits - 1)) finish_part(nunits - 1);
#undef DFMI_PSEL
}

// ---------------------------------------------------------------------------
// host side

struct PPlan {
  int U, S, T, G;
  size_t ws_bytes;
};

// Shapes the persistent kernel takes: M <= 16, int4, K a multiple of 256 with
// at least two steps, every matrix's packed weights under 2 GiB.
static bool persist_eligible(int64_t M, int64_t K, const int64_t* Ns, int nseg, int gs,
                             int bits) {
  if (M < 1 || M > 16 || bits != 4 || K % 256 != 0 || K < 512 || K >= (1ll << 24)) return false;
  if (gs != 32 && gs != 64 && gs != 128) return false;
  if (K % (8 * gs) != 0) return false;
  if (nseg < 1 || nseg > kPMaxSeg) return false;
  for (int i = 0; i < nseg; ++i)
    if (Ns[i] < 1 || Ns[i] * (K / 2) >= (1ll << 31)) return false;
  return true;
}

// Stream-K partition (see the header comment): G workgroups (two per CU, at
// least two steps each), and every workgroup's range inside one block must
// fit one scale / bias window unless whole blocks do.
static bool plan_persist(int64_t M, int64_t K, const int64_t* Ns, int nseg, int gs, PPlan& p) {
  int64_t U = 0;
  for (int i = 0; i < nseg; ++i) U += (Ns[i] + kStreamRows - 1) / kStreamRows;
  if (U > kPMaxBlocks) return false;
  p.U = (int)U;
  p.S = (int)(K / 256);
  const int64_t T = U * p.S;
  if (T >= (1ll << 31) / kPGroups) return false;
  p.T = (int)T;
  p.G = (int)std::min<int64_t>(kPGroups, std::max<int64_t>(1, T / 2));
  const int maxg = sb_max_groups(kSbPieces);
  const int step_groups = 256 / gs;
  const int64_t per = (T + p.G - 1) / p.G;  // longest range, in steps
  if ((int64_t)p.S * step_groups > maxg && per * step_groups > maxg) return false;
  p.ws_bytes = kPCounterBytes + (size_t)p.G * 2 * 16 * 64 * sizeof(float);
  (void)M;
  return true;
}

template <typename Tag, int GS, int NSEG>
static void launch_persist_n(const PArgs& a, int grid, hipStream_t st) {
  using LY = PLayout<Tag, GS>;
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&qmm_persist_kernel<Tag, GS, NSEG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, LY::BYTES);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL((qmm_persist_kernel<Tag, GS, NSEG>), dim3(grid), dim3(64 * kPWaves),
                     LY::BYTES, st, a);
}

template <typename Tag, int GS>
static void launch_persist_t(const PArgs& a, int nseg, int grid, hipStream_t st) {
  if (nseg == 1) launch_persist_n<Tag, GS, 1>(a, grid, st);
  else if (nseg == 2) launch_persist_n<Tag, GS, 2>(a, grid, st);
  else launch_persist_n<Tag, GS, 3>(a, grid, st);
}

template <typename Tag>
static void launch_persist(const PArgs& a, int nseg, int gs, int grid, hipStream_t st) {
  if (gs == 32) launch_persist_t<Tag, 32>(a, nseg, grid, st);
  else if (gs == 64) launch_persist_t<Tag, 64>(a, nseg, grid, st);
  else launch_persist_t<Tag, 128>(a, nseg, grid, st);
}

}  // namespace dfmi

using namespace dfmi;

// Plan query of the persistent kernel (dfmi_qmm.hip routes plain calls here).
bool dfmi_persist_plan(int64_t M, int64_t K, const int64_t* Ns, int nseg, int gs, int bits,
                       size_t* ws_bytes) {
  if (!persist_eligible(M, K, Ns, nseg, gs, bits)) return false;
  PPlan p;
  if (!plan_persist(M, K, Ns, nseg, gs, p)) return false;
  if (ws_bytes) *ws_bytes = p.ws_bytes;
  return true;
}

int dfmi_persist_launch(const void* x, int x_dtype, const dfmi_qmm_segment* segs, int nseg,
                        int64_t M, int64_t K, int gs, void* workspace, size_t workspace_bytes,
                        void* stream) {
  if (nseg < 1 || nseg > kPMaxSeg) {
    set_error("dfmi_qmm: %d matrices outside the persistent kernel (1..%d)", nseg, kPMaxSeg);
    return DFMI_EINVAL;
  }
  int64_t Ns[kPMaxSeg];
  for (int i = 0; i < nseg; ++i) Ns[i] = segs[i].N;
  PPlan p;
  if (!persist_eligible(M, K, Ns, nseg, gs, 4) || !plan_persist(M, K, Ns, nseg, gs, p)) {
    set_error("dfmi_qmm: shape M=%lld K=%lld outside the persistent kernel", (long long)M,
              (long long)K);
    return DFMI_EINVAL;
  }
  PArgs a;
  a.x = static_cast<const uint16_t*>(x);
  int blk = 0;
  for (int i = 0; i < kPMaxSeg; ++i) {
    if (i < nseg) {
      a.seg[i].w = segs[i].w_q;
      a.seg[i].s = static_cast<const uint16_t*>(segs[i].scales);
      a.seg[i].b = static_cast<const uint16_t*>(segs[i].biases);
      a.seg[i].y = static_cast<uint16_t*>(segs[i].y);
      a.seg[i].N = (int)segs[i].N;
      a.seg[i].blk0 = blk;
      blk += (int)((segs[i].N + kStreamRows - 1) / kStreamRows);
    } else {
      a.seg[i] = a.seg[0];
      a.seg[i].blk0 = 0x7FFFFFFF;
    }
  }
  if (!workspace || workspace_bytes < p.ws_bytes || !aligned16(workspace)) {
    set_error("dfmi_qmm: workspace of %zu bytes (16-byte aligned) required, got %zu",
              p.ws_bytes, workspace_bytes);
    return DFMI_ENOSPC;
  }
  a.counters = static_cast<uint32_t*>(workspace);
  a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + kPCounterBytes);
  a.M = (int)M;
  a.K = (int)K;
  a.S = p.S;
  a.T = p.T;
  a.G = p.G;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == DFMI_BF16) launch_persist<BF16>(a, nseg, gs, p.G, st);
  else launch_persist<F16>(a, nseg, gs, p.G, st);
  return check_launch("dfmi_qmm_persist");
}
