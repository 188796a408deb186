// 8-bit affine qmm on gfx950: y[M,N] = x[M,K] . dequant(W)^T with
// w_q uint32 [N, K/4], byte i of word j = k 4j+i (dflash_mlx/verify_qmm.py:593-598,
// the layout of the reference's mma2big_8bit / mma2big_pipe_8bit kernels).
//
// Arithmetic: a byte q = lo + 16 hi is split into its two nibble planes, each
// turned into the exact 16-bit value OFF + nibble (the same magic-number trick
// as the int4 kernels), and multiplied by the unconverted activations in one
// 16x16x32 MFMA per plane:
//   P_lo = sum x (OFF + lo),  P_hi = sum x (OFF + hi),  X = sum x
//   sum x (q s + b) = s P_lo + 16 s P_hi + (b - 17 OFF s) X      (per group)
// every product exact, every sum fp32.
//
// Launch: grid (N / (16 NT), ceil(M / 16)); a workgroup owns 16 NT weight rows
// and 16 activation rows; its wavefronts split K in 32-k blocks (whole groups
// per wavefront) and sum their partial tiles through LDS.  Register loads (no
// LDS staging): this is the general-shape path for 8-bit weights.
#include <algorithm>

#include "dfmi_device.h"
#include "dfmi_host.h"

namespace dfmi {

constexpr int k8MaxWaves = 8;

struct Qmm8Args {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int M, K, N;
};

// Two words (8 bytes = k 0..7) -> the low-nibble and high-nibble planes as
// MFMA operands of 8 values OFF + nibble in k order.
template <typename Tag>
__device__ inline void dequant8_planes(uint32_t w0, uint32_t w1, const DqConst& dq, u32x4& lo,
                                       u32x4& hi) {
  const uint32_t e0 = w0 & 0x0F0F0F0Fu, e1 = w1 & 0x0F0F0F0Fu;
  const uint32_t o0 = (w0 >> 4) & 0x0F0F0F0Fu, o1 = (w1 >> 4) & 0x0F0F0F0Fu;
  // __builtin_amdgcn_perm(S0, S1, sel): selector byte 0..3 picks a byte of S1,
  // 4..7 of S0; S0 = MAGIC supplies the high byte of each 16-bit value.
  lo.x = __builtin_amdgcn_perm(dq.magic, e0, 0x07010500u);
  lo.y = __builtin_amdgcn_perm(dq.magic, e0, 0x07030502u);
  lo.z = __builtin_amdgcn_perm(dq.magic, e1, 0x07010500u);
  lo.w = __builtin_amdgcn_perm(dq.magic, e1, 0x07030502u);
  hi.x = __builtin_amdgcn_perm(dq.magic, o0, 0x07010500u);
  hi.y = __builtin_amdgcn_perm(dq.magic, o0, 0x07030502u);
  hi.z = __builtin_amdgcn_perm(dq.magic, o1, 0x07010500u);
  hi.w = __builtin_amdgcn_perm(dq.magic, o1, 0x07030502u);
}

template <typename Tag, int GS, int NT>
__global__ __launch_bounds__(k8MaxWaves * 64) void qmm8_kernel(Qmm8Args a) {
  constexpr int BPG = GS / 32;  // 32-k blocks per group
  __shared__ float red[k8MaxWaves][NT][4][64];
  const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  const int m0 = blockIdx.y * 16;
  const int groups = a.K / GS;
  const int g0 = (int)((int64_t)wave * groups / waves);
  const int g1 = (int)((int64_t)(wave + 1) * groups / waves);
  const DqConst dq = dq_const<Tag>();
  const u32x4 ones = u32x4{Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2, Num<Tag>::ONE2};

  // activation row of this lane (rows >= M repeat row M-1; never stored)
  const uint16_t* xr = a.x + (int64_t)min(m0 + col, a.M - 1) * a.K;
  const uint32_t* wr[NT];
  const uint16_t* sr[NT];
  const uint16_t* br[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = min(n0 + 16 * t + col, a.N - 1);
    wr[t] = a.w + (int64_t)n * (a.K / 4);
    sr[t] = a.s + (int64_t)n * groups;
    br[t] = a.b + (int64_t)n * groups;
  }

  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = zero4();
  for (int g = g0; g < g1; ++g) {
    f32x4 plo[NT], phi[NT], xs = zero4();
#pragma unroll
    for (int t = 0; t < NT; ++t) plo[t] = phi[t] = zero4();
#pragma unroll
    for (int bb = 0; bb < BPG; ++bb) {
      const int k = g * GS + bb * 32 + kg * 8;  // this lane's 8 k values
      const u32x4 xa = *reinterpret_cast<const u32x4*>(xr + k);
      xs = Num<Tag>::mma(xa, ones, xs);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const u32x2 wv = *reinterpret_cast<const u32x2*>(wr[t] + k / 4);
        u32x4 lo, hi;
        dequant8_planes<Tag>(wv.x, wv.y, dq, lo, hi);
        plo[t] = Num<Tag>::mma(xa, lo, plo[t]);
        phi[t] = Num<Tag>::mma(xa, hi, phi[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float s = Num<Tag>::h2f(sr[t][g]);
      const float s16 = 16.0f * s;
      const float bq = __builtin_fmaf(-17.0f * Num<Tag>::OFF, s, Num<Tag>::h2f(br[t][g]));
#pragma unroll
      for (int r = 0; r < 4; ++r)
        acc[t][r] = __builtin_fmaf(bq, xs[r],
                                   __builtin_fmaf(s16, phi[t][r], __builtin_fmaf(s, plo[t][r], acc[t][r])));
    }
  }

#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][t][j][lane] = acc[t][j];
  __syncthreads();
  for (int e = tid; e < NT * 4 * 64; e += waves * 64) {
    const int l = e & 63, j = (e >> 6) & 3, t = e >> 8;
    float v = 0.f;
    for (int w = 0; w < waves; ++w) v += red[w][t][j][l];
    const int m = m0 + 4 * (l >> 4) + j, n = n0 + 16 * t + (l & 15);
    if (m < a.M && n < a.N) a.y[(int64_t)m * a.N + n] = Num<Tag>::f2h(v);
  }
}

template <typename Tag, int GS>
static void launch8_gs(int nt, dim3 grid, int waves, hipStream_t st, const Qmm8Args& a) {
  if (nt == 1) hipLaunchKernelGGL((qmm8_kernel<Tag, GS, 1>), grid, dim3(64 * waves), 0, st, a);
  else hipLaunchKernelGGL((qmm8_kernel<Tag, GS, 2>), grid, dim3(64 * waves), 0, st, a);
}

template <typename Tag>
static void launch8(int gs, int nt, dim3 grid, int waves, hipStream_t st, const Qmm8Args& a) {
  if (gs == 32) launch8_gs<Tag, 32>(nt, grid, waves, st, a);
  else if (gs == 64) launch8_gs<Tag, 64>(nt, grid, waves, st, a);
  else launch8_gs<Tag, 128>(nt, grid, waves, st, a);
}

}  // namespace dfmi

using namespace dfmi;

// Called by dfmi_qmm_affine_ex for bits == 8 (the shape / dtype / alignment
// checks are done there).
int dfmi_qmm8_launch(const void* x, int x_dtype, const uint32_t* w_q, const void* scales,
                     const void* biases, void* y, int64_t M, int64_t K, int64_t N, int gs,
                     void* stream) {
  Qmm8Args a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = w_q;
  a.s = static_cast<const uint16_t*>(scales);
  a.b = static_cast<const uint16_t*>(biases);
  a.y = static_cast<uint16_t*>(y);
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  const int groups = (int)(K / gs);
  const int waves = std::max(1, std::min(k8MaxWaves, groups));
  const int nt = N >= 2048 ? 2 : 1;
  const dim3 grid((unsigned)((N + 16 * nt - 1) / (16 * nt)), (unsigned)((M + 15) / 16));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == DFMI_BF16) launch8<BF16>(gs, nt, grid, waves, st, a);
  else launch8<F16>(gs, nt, grid, waves, st, a);
  return check_launch("dfmi_qmm_affine (8-bit)");
}
