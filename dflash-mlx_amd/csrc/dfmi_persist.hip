// Persistent wide streaming matmul: y_i[M, N_i] = x[M, K] . dequant(W_i)^T for
// up to four weight matrices W_i that share the activations x (one matrix for
// a plain verify linear; the q/k/v or gate/up siblings of a layer in one
// launch).  M <= 16, int4, K % 256 == 0, K a multiple of 8 groups.
//
// Why wide: every 256-k step of a block reads a 16 x 256 activation tile
// (8 KiB) besides its weights, and a CU's vector memory pipeline is bound by
// the requests it issues, not by where they hit: with 64-row blocks the
// activation requests equal the weight requests (MI355X, pure LDS-DMA
// streaming of a 389 MB matrix: 6.1 TB/s without activation traffic, 4.9
// with 1:1, 5.8 with 1:2; replicating or staggering the activations does not
// help).  Here a block is 128 rows: 8 wavefronts in two row groups of four
// (Stream<..., RW = 2>) share one activation stage, halving its requests.  One
// workgroup per CU (160 KB of LDS): four LDS stages of 24 KB (three steps in
// flight) and two scale / bias window buffers of 32 KB.
//
// Work is cut into units of one 128-row block of one matrix over a K range.
// Each workgroup streams its list of units through ONE pipeline (three steps
// ahead), across unit boundaries, so no workgroup pays more than one
// pipeline fill.
//
// Scale / bias windows: a unit's K range is cut into window segments at the
// unit's start and at every multiple of 64 groups (WSTEPS steps), so a
// segment's window is at most 8 pieces of 8 groups per row and array (32 KB
// for 128 rows, whole lines of each row).  Two buffers: the window of
// segment s + 1 is fetched as soon as the fragment reads enter segment s
// (segment s - 1's buffer is then free), so it is in flight while segment s
// computes and its wait is normally already satisfied.
//
// Work partition (stream-K in eight groups): group x = the workgroups g with
// g % 8 = x (the XCD that round-robin dispatch would give them; measured
// placement does not always follow it, and nothing relies on it) owns the
// whole blocks [x B / 8, (x + 1) B / 8) and their T_x = B_x S block-steps;
// its G_x = min(32, T_x) workgroups take contiguous ranges
// [q T_x / G_x, (q + 1) T_x / G_x).  Blocks wholly inside a range are stored
// directly; a range starts and ends with at most one partial block each, all
// of a partial block's workgroups being in one group.  A partial block's fp32
// tile goes to the workspace (slot 0 for the workgroup's first unit, slot 1
// for its last) with agent-scope atomic stores; at its end the workgroup
// waits for its own stores (vmcnt 0) and bumps the counters of its partial
// blocks with agent-scope RMWs; the last workgroup to arrive (its RMW returned
// the final count) sums the parts in workgroup order (deterministic) with
// agent-scope atomic loads issued after that return, and writes y.
// Agent-scope atomic accesses are coherent across the XCDs' L2s, so the
// exchange is correct wherever the workgroups run.  Nothing is in flight at
// the end, so the exchange never drains the pipeline.
//
// Per-unit epilogue: the 8 wavefronts' partial tiles are summed through the
// window buffer of the segment that just ended (every wavefront has read its
// last fragment of it by the wait that starts the step); the next window is
// fetched into that buffer after the sums are read.
//
// Wait accounting: every wavefront issues the same DMA instructions per step
// (Stream::CHUNK_DMA) and per window (Stream::SB_DMA), in the same order, so
// the number of loads issued after any given one is known exactly: before
// reading position q the wait leaves in flight only what was issued after
// both q's chunk and q's window.  The marks move once per position, also
// past the range (the count so far), so the wait for position p + 1 always
// reads its own mark.  Epilogue stores are left out of the count: a store
// can only lengthen a wait.
#include <algorithm>

#include "dfmi_host.h"
#include "dfmi_stream.h"

namespace dfmi {

constexpr int kPMaxSeg = 4;
constexpr int kPWaves = 8;
constexpr int kPXcds = 8;
constexpr int kPPerXcd = 32;                   // workgroups per XCD: one per CU
constexpr int kPGroups = kPXcds * kPPerXcd;    // 256
constexpr int kPSbpc = 8;                      // window pieces: 64 groups
constexpr size_t kPCounterBytes = 65536;       // one counter per block
constexpr int kPMaxBlocks = (int)(kPCounterBytes / 4);
constexpr int kPRows = 2 * kStreamRows;        // 128 rows per block
constexpr int kPPartFloats = 16 * kPRows;      // one partial tile

struct PSeg {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int N;     // rows of this matrix
  int blk0;  // first block of this matrix (blocks past the last matrix: never)
};

struct PArgs {
  const uint16_t* x;
  PSeg seg[kPMaxSeg];
  float* partials;     // partial blocks: [workgroup][2][16][128] fp32
  uint32_t* counters;  // [block], zero between calls
  int M, K;
  int S;  // 256-k steps of K
  int B;  // blocks of the launch
};

template <typename Tag, int GS>
struct PLayout {
  using S = Stream<Tag, GS, 1, kPWaves, kPSbpc, 4, 2>;
  static_assert(S::NB == kPRows && S::DEPTH == 4 && S::CK == 256, "wide stream");
  static constexpr int WIN1 = S::LDS_BYTES;  // window buffer 1 past the stream's own layout
  static constexpr int BYTES = S::LDS_BYTES + S::SBBUF;
  static_assert(BYTES <= 160 * 1024, "one workgroup per CU");
  static_assert(S::SB_OFF == 0, "window 0 at the start");
  static constexpr int WSTEPS = 8 * kPSbpc / S::GPC;  // steps of an aligned window segment
  static_assert(kPWaves * S::RED_FLOATS * 4 <= S::SBBUF, "epilogue through one window buffer");
  static_assert(4 * S::CHUNK_DMA + 2 * S::SB_DMA <= 23, "waits in range");
};

// LDS reads and writes done, then the workgroup barrier; loads stay in flight.
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // vmcnt 63, lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// stage_barrier<n> for a runtime n in 0..23 (larger: 23, waiting longer is safe)
__device__ inline void wait_loads(int n) {
  switch (n < 0 ? 0 : (n > 23 ? 23 : n)) {
#define DFMI_W(k) \
  case k: stage_barrier<k>(); break;
    DFMI_W(0) DFMI_W(1) DFMI_W(2) DFMI_W(3) DFMI_W(4) DFMI_W(5) DFMI_W(6) DFMI_W(7)
    DFMI_W(8) DFMI_W(9) DFMI_W(10) DFMI_W(11) DFMI_W(12) DFMI_W(13) DFMI_W(14) DFMI_W(15)
    DFMI_W(16) DFMI_W(17) DFMI_W(18) DFMI_W(19) DFMI_W(20) DFMI_W(21) DFMI_W(22)
#undef DFMI_W
    default: stage_barrier<23>(); break;
  }
}

// The kernel's argument block in the kernel-argument segment (constant
// memory): the matrix of a block is looked up there with a wave-uniform
// index, i.e. by scalar loads, rather than chosen among copies in registers
// (a run-time choice among copies is turned into a table in scratch memory).
typedef const __attribute__((address_space(4))) PArgs* PArgsPtr;

// One workgroup's work: its range of block-steps, the matrices, and the
// pipeline's cursors.  A plain object whose force-inlined members touch its
// fields directly, so the compiler keeps all of it in registers.
template <typename Tag, int GS>
struct PWork {
  using LY = PLayout<Tag, GS>;
  using S = typename LY::S;
  static constexpr int NT = 64 * kPWaves;
  static constexpr int D = S::DEPTH;
  static constexpr int WST = LY::WSTEPS;
  static constexpr int PER = 2 * S::RED_FLOATS / NT;  // outputs per thread of a unit

  PArgsPtr pa;  // the matrices (past the last: blk0 = INT_MAX)
  __amdgpu_buffer_rsrc_t xr;
  float* apart;
  uint32_t* acnt;
  int tid, lane, wave, g, xcd;
  int K, M, Sfull, groups;
  // this XCD's first block and block-steps, its workgroups, this range
  int bx0, Tx, Gx, t0, t1, V, u0, nunits, first_c0, last_c1;
  DqConst dq;
  typename S::Lane L;
  int ops;                 // DMA instructions this wavefront has issued
  int m0, m1, m2, m3;      // loads issued up to the chunks of positions p .. p + 3
  int mw0, mw1;            // loads issued up to the window in buffer 0 / 1
  int ij, ic;              // chunk issue cursor (unit, step)
  int wj, wc, wn;          // window issue cursor (unit, first step) and segment number
  int rj, rc, rn, rs;      // read cursor (unit, step), its segment's number and first step
  f32x4 acc[S::NT][1];

  __device__ __forceinline__ int unit_c0(int j) const { return j == 0 ? first_c0 : 0; }
  __device__ __forceinline__ int unit_c1(int j) const {
    return j == nunits - 1 ? last_c1 : Sfull;
  }
  // a unit other workgroups also work on
  __device__ __forceinline__ bool is_part(int j) const {
    return unit_c0(j) != 0 || unit_c1(j) != Sfull;
  }
  // local index of the workgroup whose range holds block-step t of this XCD
  __device__ __forceinline__ int owner(int t) const {
    return (int)(((int64_t)(t + 1) * Gx - 1) / Tx);
  }
  // the matrix holding block u: the last whose first block is at most u
  __device__ __forceinline__ int seg_of(int u) const {
    return __builtin_amdgcn_readfirstlane((int)(u >= pa->seg[1].blk0) +
                                          (int)(u >= pa->seg[2].blk0) +
                                          (int)(u >= pa->seg[3].blk0));
  }
  // end of the window segment that starts at step c of unit j
  __device__ __forceinline__ int seg_end(int j, int c) const {
    return min(unit_c1(j), (c / WST + 1) * WST);
  }

  // false: no work for this workgroup (uniform)
  __device__ __forceinline__ bool init(const PArgs& a) {
    pa = (PArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    g = blockIdx.x;
    xcd = g % kPXcds;
    const int q = g / kPXcds;
    K = a.K;
    M = a.M;
    Sfull = a.S;
    groups = K / GS;
    bx0 = (int)((int64_t)xcd * a.B / kPXcds);
    const int bx1 = (int)((int64_t)(xcd + 1) * a.B / kPXcds);
    Tx = (bx1 - bx0) * Sfull;
    // at most one workgroup per block-step, so every range is non-empty and
    // the workgroups between a block's first and last owner all hold part of it
    Gx = min(kPPerXcd, Tx);
    if (q >= Gx) return false;
    t0 = (int)((int64_t)q * Tx / Gx);
    t1 = (int)((int64_t)(q + 1) * Tx / Gx);
    V = t1 - t0;
    u0 = bx0 + t0 / Sfull;
    nunits = (t1 - 1) / Sfull - t0 / Sfull + 1;
    first_c0 = t0 - (t0 / Sfull) * Sfull;
    last_c1 = t1 - ((t1 - 1) / Sfull) * Sfull;
    xr = buffer_rsrc(a.x, (uint32_t)M * (uint32_t)K * 2u);
    apart = a.partials;
    acnt = a.counters;
    dq = dq_const<Tag>();
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
    ops = m0 = m1 = m2 = m3 = mw0 = mw1 = 0;
    ij = 0;
    ic = unit_c0(0);
    wj = 0;
    wc = unit_c0(0);
    wn = 0;
    rj = 0;
    rc = rs = unit_c0(0);
    rn = 0;
    return true;
  }

  // unit j's context for the DMA: its matrix's buffers and first row
  __device__ __forceinline__ void unit_ctx(int j, typename S::Ctx& cx) const {
    const int u = u0 + j;
    const auto& m = pa->seg[seg_of(u)];
    const int N = m.N;
    cx.x = xr;
    cx.w = buffer_rsrc(m.w, (uint32_t)N * (uint32_t)(K / 2));
    cx.s = buffer_rsrc(m.s, (uint32_t)N * (uint32_t)groups * 2u);
    cx.b = buffer_rsrc(m.b, (uint32_t)N * (uint32_t)groups * 2u);
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
    cx.n0 = (u - m.blk0) * S::NB;
    cx.lane = lane;
    cx.wave = wave;
    cx.sb_base = 0;
  }

  // the window of the next segment, into buffer (its number & 1)
  __device__ __forceinline__ void issue_window() {
    if (wj >= nunits) return;  // uniform: no segment left
    typename S::Ctx cx;
    unit_ctx(wj, cx);
    cx.sb_base = (wn & 1) ? (uint32_t)LY::WIN1 : 0u;
    const int ce = seg_end(wj, wc);
    const int piece0 = (wc * S::GPC) >> 3;
    S::issue_sb(cx, piece0, ((ce * S::GPC + 7) >> 3) - piece0);
    ops += S::SB_DMA;
    if (wn & 1) mw1 = ops;
    else mw0 = ops;
    ++wn;
    if (ce == unit_c1(wj)) {
      ++wj;
      wc = unit_c0(wj);
    } else {
      wc = ce;
    }
  }

  // position p's chunk (p < V), then the marks move on by one position
  __device__ __forceinline__ void issue_next(int p) {
    if (p < V) {
      typename S::Ctx cx;
      unit_ctx(ij, cx);
      if (ic == unit_c0(ij)) L = S::lane_setup(cx);  // a new unit's weight rows
      S::issue_chunk(cx, L, ic, __builtin_amdgcn_readfirstlane(p % D));
      ops += S::CHUNK_DMA;
      if (++ic == unit_c1(ij)) {
        ++ij;
        ic = unit_c0(ij);
      }
    }
    m0 = m1;
    m1 = m2;
    m2 = m3;
    m3 = ops;
  }

  // wait until the read position's chunk (mark mc) and window have landed
  __device__ __forceinline__ void wait_for_read(int mc) const {
    wait_loads(ops - max(mc, (rn & 1) ? mw1 : mw0));
  }

  // fragments of position p (the read cursor) from stage p % D
  __device__ __forceinline__ void read_next(int p, typename S::Frag& f) const {
    typename S::Ctx cr;
    cr.wave = wave;
    cr.sb_base = (rn & 1) ? (uint32_t)LY::WIN1 : 0u;
    const int g0w = ((rs * S::GPC) >> 3) * 8;
    S::read_frag(cr, L, rc, __builtin_amdgcn_readfirstlane(p % D), g0w, f);
  }

  // move the read cursor on by one position; true when it entered a new
  // window segment
  __device__ __forceinline__ bool read_advance() {
    ++rc;
    if (rc == unit_c1(rj)) {
      ++rj;
      rc = unit_c0(rj);
    } else if (rc % WST != 0) {
      return false;
    }
    ++rn;
    rs = rc;
    return true;
  }

  // unit j's outputs, summed through window buffer wb (its segment ended)
  __device__ __forceinline__ void epilogue(int j, int wb) {
    const int u = u0 + j;
    const auto& m = pa->seg[seg_of(u)];
    const int N = m.N;
    uint16_t* y = m.y;
    const int n0 = (u - m.blk0) * S::NB;
    float* red = reinterpret_cast<float*>(dfmi_smem + (wb ? LY::WIN1 : 0));
    lds_barrier();  // every wavefront's last reads of that buffer are done
    {
      float* mine = red + wave * S::RED_FLOATS;
#pragma unroll
      for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mine[(t * 4 + r) * 64 + lane] = acc[t][0][r];
    }
    lds_barrier();
    float v[PER];
    int mi[PER], ni[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int el = e * NT + tid;  // 0 .. 2047
      const int rg = el / S::RED_FLOATS, eo = el % S::RED_FLOATS;
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < S::KW; ++k) sum += red[(rg * S::KW + k) * S::RED_FLOATS + eo];
      v[e] = sum;
      const int l = eo & 63, jj = (eo >> 6) & 3, t = eo >> 8;
      mi[e] = 4 * (l >> 4) + jj;
      ni[e] = 64 * rg + 16 * t + (l & 15);  // row within the block
    }
    if (!is_part(j)) {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int n = n0 + ni[e];
        if (mi[e] < M && n < N) y[(int64_t)mi[e] * N + n] = Num<Tag>::f2h(v[e]);
      }
      return;
    }
    // a partial block: its tile to this workgroup's slot, summed at the end
    float* part = apart + ((int64_t)g * 2 + (j == 0 ? 0 : 1)) * kPPartFloats;
#pragma unroll
    for (int e = 0; e < PER; ++e)
      __hip_atomic_store(part + mi[e] * kPRows + ni[e], v[e], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }

  // At the workgroup's end (nothing in flight): the exchange for a partial
  // block of unit j; the last workgroup to arrive sums the parts in
  // workgroup order and writes y.
  __device__ __forceinline__ void finish_part(int j) {
    const int u = u0 + j;
    const auto& m = pa->seg[seg_of(u)];
    const int N = m.N;
    uint16_t* y = m.y;
    const int n0 = (u - m.blk0) * S::NB;
    const int tb = (u - bx0) * Sfull;  // the block's first block-step in this XCD
    const int wf = owner(tb), wl = owner(tb + Sfull - 1);
    int* s_last = reinterpret_cast<int*>(dfmi_smem);
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
    for (int e = 0; e < PER; ++e) {
      const int el = e * NT + tid;
      const int rg = el / S::RED_FLOATS, eo = el % S::RED_FLOATS;
      const int l = eo & 63, jj = (eo >> 6) & 3;
      mi[e] = 4 * (l >> 4) + jj;
      ni[e] = 64 * rg + 16 * (eo >> 8) + (l & 15);
      sum[e] = 0.f;
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
        const int slot = ((int)((int64_t)v * Tx / Gx) / Sfull == u - bx0) ? 0 : 1;
        const float* src = apart + ((int64_t)(v * kPXcds + xcd) * 2 + slot) * kPPartFloats;
#pragma unroll
        for (int e = 0; e < PER; ++e)
          t4[i][e] = __hip_atomic_load(src + mi[e] * kPRows + ni[e], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < PER; ++e) sum[e] += (v0 + i <= wl) ? t4[i][e] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int n = n0 + ni[e];
      if (mi[e] < M && n < N) y[(int64_t)mi[e] * N + n] = Num<Tag>::f2h(sum[e]);
    }
    if (tid == 0)
      __hip_atomic_exchange(&acnt[u], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // iteration p: position p's fragments are in cur.  Wait for position p + 1
  // (chunk and window), fetch position p + 4 into p's stage, read p + 1;
  // compute p; at a unit's end its epilogue; when the read of p + 1 entered a
  // window segment, fetch the window after it into the buffer p's segment
  // just freed.  (cj, cc, cn): compute cursor and its segment.
  __device__ __forceinline__ void step(int p, typename S::Frag& cur, typename S::Frag& nxt,
                                       bool& entered, int& cj, int& cc, int& cn) {
    const bool last = cc == unit_c1(cj) - 1;
    if (p + 1 < V) {
      wait_for_read(m1);
      issue_next(p + D);
      read_next(p + 1, nxt);
    }
    if (cc == unit_c0(cj)) {
#pragma unroll
      for (int t = 0; t < S::NT; ++t) acc[t][0] = zero4();
    }
    S::compute(L, cur, acc, dq);
    if (last) epilogue(cj, cn & 1);  // through the buffer of p's segment
    if (p + 1 < V && entered) {
      if (last) lds_barrier();  // the epilogue's reads of that buffer are done
      issue_window();
    }
    if (p + 1 < V) entered = read_advance();
    if (++cc == unit_c1(cj)) {
      ++cj;
      cc = unit_c0(cj);
      ++cn;
    } else if (cc % WST == 0) {
      ++cn;
    }
  }

  __device__ __forceinline__ void run() {
    // prologue: the first two windows (both buffers free), then positions 0..3
    issue_window();
    issue_window();
#pragma unroll
    for (int k = 0; k < D; ++k) issue_next(k);
    typename S::Frag fa, fb;
    wait_for_read(m0);  // position 0 and window 0 landed
    read_next(0, fa);
    bool entered = read_advance();
    int cj = 0, cc = unit_c0(0), cn = 0;
    int p = 0;
    for (; p + 1 < V; p += 2) {
      step(p, fa, fb, entered, cj, cc, cn);
      step(p + 1, fb, fa, entered, cj, cc, cn);
    }
    if (p < V) step(p, fa, fb, entered, cj, cc, cn);
    if (is_part(0)) finish_part(0);
    if (nunits > 1 && is_part(nunits - 1)) finish_part(nunits - 1);
  }
};

template <typename Tag, int GS>
__global__ __launch_bounds__(64 * kPWaves) void qmm_persist_kernel(PArgs a) {
  PWork<Tag, GS> w;
  if (!w.init(a)) return;  // uniform
  w.run();
}

// ---------------------------------------------------------------------------
// host side

struct PPlan {
  int B, S;
  size_t ws_bytes;
};

// Shapes the persistent kernel takes: M <= 16, int4, K a multiple of 256 and
// of 8 groups, every matrix's packed weights under 2 GiB, at most 16384
// blocks of 128 rows.
static bool plan_persist(int64_t M, int64_t K, const int64_t* Ns, int nseg, int gs, int bits,
                         PPlan& p) {
  if (M < 1 || M > 16 || bits != 4 || K % 256 != 0 || K < 256 || K >= (1ll << 24)) return false;
  if (gs != 32 && gs != 64 && gs != 128) return false;
  if (K % (8 * gs) != 0) return false;
  if (nseg < 1 || nseg > kPMaxSeg) return false;
  int64_t B = 0;
  for (int i = 0; i < nseg; ++i) {
    if (Ns[i] < 0 || Ns[i] * (K / 2) >= (1ll << 31)) return false;
    B += (Ns[i] + kPRows - 1) / kPRows;
  }
  if (B < 1 || B > kPMaxBlocks) return false;
  if ((B / kPXcds + 1) * (K / 256) * kPPerXcd >= (1ll << 31)) return false;
  p.B = (int)B;
  p.S = (int)(K / 256);
  p.ws_bytes = kPCounterBytes + (size_t)kPGroups * 2 * kPPartFloats * sizeof(float);
  return true;
}

template <typename Tag, int GS>
static void launch_persist_t(const PArgs& a, hipStream_t st) {
  using LY = PLayout<Tag, GS>;
  static const bool attr = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&qmm_persist_kernel<Tag, GS>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, LY::BYTES);
    return true;
  }();
  (void)attr;
  hipLaunchKernelGGL((qmm_persist_kernel<Tag, GS>), dim3(kPGroups), dim3(64 * kPWaves), LY::BYTES,
                     st, a);
}

template <typename Tag>
static void launch_persist(const PArgs& a, int gs, hipStream_t st) {
  if (gs == 32) launch_persist_t<Tag, 32>(a, st);
  else if (gs == 64) launch_persist_t<Tag, 64>(a, st);
  else launch_persist_t<Tag, 128>(a, st);
}

}  // namespace dfmi

using namespace dfmi;

// Plan query of the persistent kernel (dfmi_qmm.hip routes calls here).
bool dfmi_persist_plan(int64_t M, int64_t K, const int64_t* Ns, int nseg, int gs, int bits,
                       size_t* ws_bytes) {
  PPlan p;
  if (!plan_persist(M, K, Ns, nseg, gs, bits, p)) return false;
  if (ws_bytes) *ws_bytes = p.ws_bytes;
  return true;
}

int dfmi_persist_launch(const void* x, int x_dtype, const dfmi_qmm_segment* segs, int nseg,
                        int64_t M, int64_t K, int gs, void* workspace, size_t workspace_bytes,
                        void* stream) {
  int64_t Ns[kPMaxSeg];
  PPlan p;
  if (nseg >= 1 && nseg <= kPMaxSeg)
    for (int i = 0; i < nseg; ++i) Ns[i] = segs[i].N;
  if (nseg < 1 || nseg > kPMaxSeg || !plan_persist(M, K, Ns, nseg, gs, 4, p)) {
    set_error("dfmi_qmm: shape M=%lld K=%lld (%d matrices) outside the persistent kernel",
              (long long)M, (long long)K, nseg);
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
      blk += (int)((segs[i].N + kPRows - 1) / kPRows);
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
  a.B = p.B;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == DFMI_BF16) launch_persist<BF16>(a, gs, st);
  else launch_persist<F16>(a, gs, st);
  return check_launch("dfmi_qmm_persist");
}
