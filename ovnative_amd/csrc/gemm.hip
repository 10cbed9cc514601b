// int8 x int8 MFMA GEMM with the reference's per-block epilogue, for gfx950.
//
// Reference arithmetic (cpp/src/backend/cpu/gemm.cpp:432-504, per output):
//   acc_b = sum_{k in block b} q[m,k] * w[n,k]                 (exact int32)
//   f     = fma((float)acc_b, asc[m,b], f)   for b = 0 .. Kb-1 (f starts at +0)
//   C     = f * wscale[n]             (then C_old + that, rounded separately)
//
// Mapping onto the matrix cores: one V_MFMA_I32_32X32X32_I8 consumes exactly one
// 32-k block, so its int32 result IS acc_b for a 32x32 output tile.  Weight rows
// n are the MFMA's A operand (output rows i) and activation rows m its B operand
// (output columns j = lane % 32).  A lane then holds 16 accumulators of ONE
// activation row m, so the block scale asc[m,b] is one register per lane and the
// per-block epilogue is 16 x (cvt, fma) on values already in registers; wscale
// is applied once after the K loop.
//
// Tiles: a workgroup computes BN weight rows x BM activation rows with WN x WM
// wavefronts; K is staged through LDS two blocks (64 bytes) at a time, global
// loads of the next stage in flight while the current one is multiplied.
#include "gemm.h"
#include "ovh_common.h"

namespace ovh {

namespace {

constexpr int KC = 64;          // K bytes per LDS stage (2 blocks)
constexpr int LDSS = KC + 16;   // padded LDS row stride (bytes)

__device__ __forceinline__ i32x16 mfma_i8(i32x4 a, i32x4 b) {
  const i32x16 z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

template <int BN, int BM, int WN, int WM, int MODE>
__global__ __launch_bounds__(64 * WN * WM) void gemm_i8_kernel(const GemmArgs a) {
  constexpr int NT = 64 * WN * WM;
  constexpr int TN = BN / WN, TM = BM / WM;
  constexpr int FN = TN / 32, FM = TM / 32;
  static_assert(FN >= 1 && FM >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  constexpr int WCH = BN * (KC / 16), ACH = BM * (KC / 16);  // 16-byte chunks per stage
  constexpr int WPT = (WCH + NT - 1) / NT, APT = (ACH + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) int8_t sW[BN * LDSS];
  __shared__ __attribute__((aligned(16))) int8_t sA[BM * LDSS];
  __shared__ float sS[BM][KC / 32];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WN, wm = wave / WN;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int64_t Kp = a.Kp;

  f32x16 f[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) f[i][j][e] = 0.f;

  i32x4 wreg[WPT], areg[APT];
  float sreg = 0.f;

  auto gload = [&](int64_t kc) {
#pragma unroll
    for (int t = 0; t < WPT; ++t) {
      const int c = tid + t * NT;
      const int r = c / (KC / 16), col = c % (KC / 16);
      const int64_t k = kc + col * 16;
      i32x4 v = {0, 0, 0, 0};
      if (c < WCH && k < Kp) v = *reinterpret_cast<const i32x4*>(a.W + (int64_t)(n0 + r) * Kp + k);
      wreg[t] = v;
    }
#pragma unroll
    for (int t = 0; t < APT; ++t) {
      const int c = tid + t * NT;
      const int r = c / (KC / 16), col = c % (KC / 16);
      const int64_t k = kc + col * 16;
      i32x4 v = {0, 0, 0, 0};
      if (c < ACH && k < Kp && m0 + r < a.M)
        v = *reinterpret_cast<const i32x4*>(a.aq + (int64_t)(m0 + r) * Kp + k);
      areg[t] = v;
    }
    if (MODE != kDumpBlocks && tid < BM * (KC / 32)) {
      const int r = tid / (KC / 32), bb = tid % (KC / 32);
      const int64_t b = kc / 32 + bb;
      sreg = (m0 + r < a.M && b < a.Kb) ? a.asc[(int64_t)(m0 + r) * a.Kb + b] : 0.f;
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int t = 0; t < WPT; ++t) {
      const int c = tid + t * NT;
      if (c < WCH) {
        const int r = c / (KC / 16), col = c % (KC / 16);
        *reinterpret_cast<i32x4*>(sW + r * LDSS + col * 16) = wreg[t];
      }
    }
#pragma unroll
    for (int t = 0; t < APT; ++t) {
      const int c = tid + t * NT;
      if (c < ACH) {
        const int r = c / (KC / 16), col = c % (KC / 16);
        *reinterpret_cast<i32x4*>(sA + r * LDSS + col * 16) = areg[t];
      }
    }
    if (tid < BM * (KC / 32)) sS[tid / (KC / 32)][tid % (KC / 32)] = sreg;
  };

  gload(0);
  for (int64_t kc = 0; kc < Kp; kc += KC) {
    __syncthreads();  // previous stage fully consumed
    sstore();
    __syncthreads();
    if (kc + KC < Kp) gload(kc + KC);  // next stage's loads overlap this stage's math
    const int nblk = (Kp - kc) >= KC ? 2 : 1;
    for (int bb = 0; bb < nblk; ++bb) {
      i32x4 af[FN], bf[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i)
        af[i] = *reinterpret_cast<const i32x4*>(sW + (wn * TN + i * 32 + (lane & 31)) * LDSS +
                                                bb * 32 + (lane >> 5) * 16);
#pragma unroll
      for (int j = 0; j < FM; ++j)
        bf[j] = *reinterpret_cast<const i32x4*>(sA + (wm * TM + j * 32 + (lane & 31)) * LDSS +
                                                bb * 32 + (lane >> 5) * 16);
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const float s = sS[wm * TM + j * 32 + (lane & 31)][bb];
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          const i32x16 acc = mfma_i8(af[i], bf[j]);
          if (MODE == kDumpBlocks) {
            const int m = m0 + wm * TM + j * 32 + (lane & 31);
            const int64_t b = kc / 32 + bb;
            if (m < a.M) {
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                const int n = n0 + wn * TN + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (n < a.N) a.dump[((int64_t)m * a.N + n) * a.Kb + b] = acc[e];
              }
            }
          } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) f[i][j][e] = fmaf((float)acc[e], s, f[i][j][e]);
          }
        }
      }
    }
  }
  if (MODE == kDumpBlocks) return;

  // Epilogue: column scale, optional residual add, slice-aware store.
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + wm * TM + j * 32 + (lane & 31);
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nb = n0 + wn * TN + i * 32 + 8 * g + 4 * (lane >> 5);
        if (nb >= a.N) continue;
        const f32x4 ws = *reinterpret_cast<const f32x4*>(a.ws + nb);
        int s = 0;
#pragma unroll
        for (int t = 1; t < kMaxSlices; ++t)
          if (t < a.nslices && nb >= a.start[t]) s = t;
        float* dst = a.out[s] + (int64_t)m * a.ld[s] + (nb - a.start[s]);
        const int lim = a.start[s + 1] - nb;  // valid columns in this group (>= 1)
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(f[i][j][4 * g + e], ws[e]);
        if (lim >= 4 && ((uintptr_t)dst & 15u) == 0) {
          f32x4 v;
          if (MODE == kAccumulate) {
            const f32x4 c = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(o[e], c[e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[e];
          }
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (e < lim) dst[e] = MODE == kAccumulate ? __fadd_rn(o[e], dst[e]) : o[e];
          }
        }
      }
    }
  }
}

template <int BN, int BM, int WN, int WM>
hipError_t launch_cfg(const GemmArgs& a, GemmMode mode, hipStream_t st, int64_t Npad) {
  const dim3 grid((unsigned)(Npad / BN), (unsigned)((a.M + BM - 1) / BM)), block(64 * WN * WM);
  switch (mode) {
    case kStore:
      hipLaunchKernelGGL((gemm_i8_kernel<BN, BM, WN, WM, kStore>), grid, block, 0, st, a);
      break;
    case kAccumulate:
      hipLaunchKernelGGL((gemm_i8_kernel<BN, BM, WN, WM, kAccumulate>), grid, block, 0, st, a);
      break;
    case kDumpBlocks:
      hipLaunchKernelGGL((gemm_i8_kernel<BN, BM, WN, WM, kDumpBlocks>), grid, block, 0, st, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const GemmArgs& a, GemmMode mode, hipStream_t st) {
  const int64_t Npad = ((int64_t)a.N + kRowPad - 1) / kRowPad * kRowPad;
  // Largest tile that still gives every CU a workgroup; the smallest otherwise.
  auto tiles = [&](int bn, int bm) { return (Npad / bn) * (((int64_t)a.M + bm - 1) / bm); };
  constexpr int64_t kCUs = 256;
  if (a.M > 64 && tiles(128, 128) >= kCUs) return launch_cfg<128, 128, 2, 2>(a, mode, st, Npad);
  if (a.M > 32 && tiles(128, 64) >= kCUs) return launch_cfg<128, 64, 2, 2>(a, mode, st, Npad);
  if (a.M > 32 && tiles(64, 64) >= kCUs) return launch_cfg<64, 64, 2, 2>(a, mode, st, Npad);
  if (tiles(64, 32) >= kCUs) return launch_cfg<64, 32, 2, 1>(a, mode, st, Npad);
  return launch_cfg<32, 32, 1, 1>(a, mode, st, Npad);
}

// ---------------------------------------------------------------------------
// Weight layout: OVW1 int8 in layout 0 ([N,K]) or 1 ([K,N]) -> [Npad][Kp] with
// zero padding; scales -> [Npad] with zeros.  Load-time only.
__global__ void weight_layout_kernel(int64_t N, int64_t K, int64_t Npad, int64_t Kp,
                                     const int8_t* __restrict__ src, int layout,
                                     int8_t* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= Npad * Kp) return;
  const int64_t n = idx / Kp, k = idx - n * Kp;
  int8_t v = 0;
  if (n < N && k < K) v = layout == 0 ? src[n * K + k] : src[k * N + n];
  dst[idx] = v;
}

__global__ void scale_pad_kernel(int64_t N, int64_t Npad, const float* __restrict__ src,
                                 float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < Npad) dst[i] = i < N ? src[i] : 0.f;
}

__global__ void weight_to_nk_kernel(int64_t N, int64_t K, int64_t Kp,
                                    const int8_t* __restrict__ src, int8_t* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * K) return;
  const int64_t n = idx / K, k = idx - n * K;
  dst[idx] = src[n * Kp + k];
}

hipError_t launch_weight_layout(int64_t N, int64_t K, const int8_t* src, int layout,
                                const float* scale_src, DeviceWeight& w, hipStream_t st) {
  const int64_t total = w.Npad * w.Kp;
  hipLaunchKernelGGL(weight_layout_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     st, N, K, w.Npad, w.Kp, src, layout, w.q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(scale_pad_kernel, dim3((unsigned)((w.Npad + 255) / 256)), dim3(256), 0, st,
                     N, w.Npad, scale_src, w.scale);
  return hipGetLastError();
}

hipError_t launch_weight_to_nk(const DeviceWeight& w, int8_t* q_nk, hipStream_t st) {
  const int64_t total = w.N * w.K;
  hipLaunchKernelGGL(weight_to_nk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     w.N, w.K, w.Kp, w.q, q_nk);
  return hipGetLastError();
}

}  // namespace ovh
