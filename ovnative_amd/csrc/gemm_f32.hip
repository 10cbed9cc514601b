// fp32 linear on the f16 matrix cores: the reference's fp32 Mat branch
// (cpp/src/model/mat.cpp:11-13 -> linear_f32_ld, cpp/src/backend/cpu/gemm.cpp:
// 884-905, micro-kernel :64-110), C[m, n] = sum_k A[m, k] W[k, n], which the
// default int8 checkpoint uses for the audio head (tools/convert_weights.py keeps
// audio_heads fp32, stored [K, N]).
//
// The reference sums each output as one fma chain over k.  Here every fp32
// operand x becomes x * 2^-e = hi + lo with hi = f16(x * 2^-e), lo =
// f16(x * 2^-e - hi), the power of two chosen per activation row and per weight
// column so that the row's (column's) largest magnitude lands in [2^14, 2^15):
// nothing overflows f16 and hi + lo carries 22 bits of every value the row
// scale does not push below f16's normal range.  Each product is hi*hi + hi*lo
// + lo*hi on V_MFMA_F32_32X32X16_F16 (lo*lo, ~2^-22 relative, is dropped), the
// sums are fp32, and the output is scaled back by 2^(e_m + e_n), exactly.
// Against the reference's chain the result differs by summation order and
// the dropped term: a few fp32 ulps of sum_k |A W| per output.
//
// Operand planes (hi and lo alike): 1 KiB fragments of 32 rows x 16 k in the
// order one lane loads for the MFMA (lane l: row l % 32, k 8 (l / 32) .. +7),
// fragments (row tile, k step) row-tile-major; rows padded to a multiple of 128
// and k to a multiple of 16, with zeros (activations: rows past M are
// whatever the producer left, and only ever reach outputs that are not stored).
#include "gemm.h"
#include "ovh_common.h"

namespace ovh {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kFrag = 512;  // halves per fragment (1 KiB)

// Half index of (row r, k) in a plane with Ks k steps.
__host__ __device__ inline int64_t plane_index(int64_t r, int64_t k, int64_t Ks) {
  return (((r >> 5) * Ks + (k >> 4)) * 64 + (r & 31) + 32 * ((k >> 3) & 1)) * 8 + (k & 7);
}

// 2^e with the row (column) maximum amax * 2^-e in [2^14, 2^15); 1 for a zero row.
__device__ __forceinline__ int pow2_exponent(float amax) {
  if (!(amax > 0.f) || !(amax < INFINITY)) return 0;
  int ex;
  (void)frexpf(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
  return ex - 15;
}

__device__ __forceinline__ void split_scaled(float v, float inv, _Float16& hi, _Float16& lo) {
  const float x = __fmul_rn(v, inv);  // a power of two: exact
  hi = (_Float16)x;
  lo = (_Float16)__fsub_rn(x, (float)hi);
}

// ---------------------------------------------------------------------------
// weights: column scales, then planes (load time only)

__global__ void f32_col_scale_kernel(int64_t N, int64_t K, const float* __restrict__ src,
                                     int layout, int64_t Np, float* __restrict__ scale) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= Np) return;
  float am = 0.f;
  if (n < N)
    for (int64_t k = 0; k < K; ++k)
      am = fmaxf(am, fabsf(layout ? src[k * N + n] : src[n * K + k]));
  scale[n] = n < N ? ldexpf(1.f, pow2_exponent(am)) : 0.f;
}

// One thread per (column n, 8 consecutive k): 16 bytes of each plane.
__global__ void f32_weight_planes_kernel(int64_t N, int64_t K, const float* __restrict__ src,
                                         int layout, int64_t Np, int64_t Ks,
                                         const float* __restrict__ scale,
                                         _Float16* __restrict__ hi, _Float16* __restrict__ lo) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t groups = Ks * 2;
  if (t >= Np * groups) return;
  const int64_t n = t / groups, k0 = (t - n * groups) * 8;
  const float inv = n < N ? __fdiv_rn(1.f, scale[n]) : 0.f;
  h8 vh, vl;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t k = k0 + i;
    const float v = (n < N && k < K) ? (layout ? src[k * N + n] : src[n * K + k]) : 0.f;
    _Float16 a, b;
    split_scaled(v, inv, a, b);
    vh[i] = a;
    vl[i] = b;
  }
  const int64_t at = plane_index(n, k0, Ks);
  *reinterpret_cast<h8*>(hi + at) = vh;
  *reinterpret_cast<h8*>(lo + at) = vl;
}

// ---------------------------------------------------------------------------
// activations

// One workgroup per padded row: the row maximum, then 8 k per thread per pass;
// rows >= M and k >= K are written as zeros.
__global__ __launch_bounds__(256) void f32_split_rows_kernel(int64_t M, int64_t K, int64_t Ks,
                                                             const float* __restrict__ A,
                                                             _Float16* __restrict__ hi,
                                                             _Float16* __restrict__ lo,
                                                             float* __restrict__ scale) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const float* row = A + (r < M ? r : 0) * K;
  float am = 0.f;
  if (r < M)
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) am = fmaxf(am, fabsf(row[k]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int e = pow2_exponent(am);
  const float inv = ldexpf(1.f, -e);
  if (threadIdx.x == 0) scale[r] = ldexpf(1.f, e);
  for (int64_t k0 = 8 * (int64_t)threadIdx.x; k0 < Ks * 16; k0 += 8 * (int64_t)blockDim.x) {
    h8 vh, vl;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = (r < M && k0 + i < K) ? row[k0 + i] : 0.f;
      _Float16 a, b;
      split_scaled(v, inv, a, b);
      vh[i] = a;
      vl[i] = b;
    }
    const int64_t at = plane_index(r, k0, Ks);
    *reinterpret_cast<h8*>(hi + at) = vh;
    *reinterpret_cast<h8*>(lo + at) = vl;
  }
}

// The final RMSNorm of the LM (rmsnorm_f32, cpp/src/backend/cpu/ops_cpu.cpp:
// 38-62, the same sum of squares as rmsnorm_quantize: eight fma chains, element
// i into chain i % 8, chains added 0..7; xn = (x * scale) * w) for rows of 256*P
// columns, one wavefront per row, its output split straight into the planes.
template <int P>
__global__ __launch_bounds__(64) void rmsnorm_split_rows_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                float eps, int64_t Ks,
                                                                _Float16* __restrict__ hi,
                                                                _Float16* __restrict__ lo,
                                                                float* __restrict__ scale) {
  constexpr int cols = 256 * P, T = cols / 8, TP = T + 4;
  __shared__ __attribute__((aligned(16))) float xt[8 * TP];
  const int lane = threadIdx.x;
  const int64_t r = blockIdx.x;
  const float* row = x + r * cols;
  f32x4 xv[P], wv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) xv[p] = *reinterpret_cast<const f32x4*>(row + 256 * p + 4 * lane);
#pragma unroll
  for (int p = 0; p < P; ++p) wv[p] = *reinterpret_cast<const f32x4*>(w + 256 * p + 4 * lane);
  // element 256p + 4l + c -> chain 4(l&1) + c, position 32p + l/2
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int c = 0; c < 4; ++c) xt[(4 * (lane & 1) + c) * TP + 32 * p + (lane >> 1)] = xv[p][c];
  __syncthreads();
  float part = 0.f;
  if (lane < 8) {
    float acc = 0.f;
#pragma unroll 8
    for (int t = 0; t < T; t += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&xt[lane * TP + t]);
      acc = fmaf(v[0], v[0], acc);
      acc = fmaf(v[1], v[1], acc);
      acc = fmaf(v[2], v[2], acc);
      acc = fmaf(v[3], v[3], acc);
    }
    part = acc;
  }
  const float sum = sum_lanes8_in_order(part);
  const float s = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)cols), eps)));
  float v[P][4];
  float am = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[p][i] = __fmul_rn(__fmul_rn(xv[p][i], s), wv[p][i]);
      am = fmaxf(am, fabsf(v[p][i]));
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
  const int e = pow2_exponent(am);
  const float inv = ldexpf(1.f, -e);
  if (lane == 0) scale[r] = ldexpf(1.f, e);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    h4 vh, vl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      _Float16 a, b;
      split_scaled(v[p][i], inv, a, b);
      vh[i] = a;
      vl[i] = b;
    }
    // k = 256p + 4 lane .. +3: four consecutive halves of one lane slot
    const int64_t at = plane_index(r, 256 * p + 4 * lane, Ks);
    *reinterpret_cast<h4*>(hi + at) = vh;
    *reinterpret_cast<h4*>(lo + at) = vl;
  }
}

// ---------------------------------------------------------------------------
// The GEMM: 128 x 128 output tiles (weight columns n x activation rows m), four
// wavefronts of 64 x 64 (2 x 2 MFMA tiles of 32 x 32); one 16-k step per LDS
// stage (8 weight and 8 activation fragments, 16 KiB), moved by
// global_load_lds_dwordx4 (each wavefront 4 fragments per stage) through an
// NST-stage ring, each wavefront waiting on its own DMA count; XCD-aware tile
// order (an XCD walks a contiguous range of weight column tiles).

__device__ __forceinline__ f32x16 mfma_h(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int NST>
__global__ __launch_bounds__(256) void gemm_f32s_kernel(const GemmF32Args a) {
  constexpr int STAGE = 16 * 1024;
  __shared__ __attribute__((aligned(16))) char smem[NST][STAGE];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave & 1, wm = wave >> 1;
  const int n_tiles = (a.N + 127) / 128;
  int nt, mt;
  if (!tile_of(blockIdx.x, n_tiles, nt, mt)) return;  // padding workgroup
  const int64_t Ks = a.Ks;
  const int nst = (int)Ks;
  // this wavefront's 4 fragments of every stage: waves 0-1 the weight
  // fragments (4 column tiles x hi/lo), waves 2-3 the activation fragments
  const _Float16* src[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int idx = wave * 4 + t;  // fragment slot in the stage: (tile, plane)
    const int tile = (idx & 7) >> 1, plane = idx & 1;
    if (idx < 8)
      src[t] = (plane ? a.wlo : a.whi) + ((int64_t)(nt * 4 + tile) * Ks) * kFrag + lane * 8;
    else
      src[t] = (plane ? a.alo : a.ahi) + ((int64_t)(mt * 4 + tile) * Ks) * kFrag + lane * 8;
  }
  auto issue = [&](int s) __attribute__((always_inline)) {
    char* base = smem[s % NST];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src[t] + (int64_t)s * kFrag),
                                       (lds_void_t*)(base + (wave * 4 + t) * 1024), 16, 0, 0);
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

#pragma unroll
  for (int s = 0; s < NST - 1; ++s)
    if (s < nst) issue(s);
  for (int s = 0; s < nst; ++s) {
    if (s + NST - 2 < nst)
      wait_vm_lgkm<4 * (NST - 2)>();
    else
      wait_vm_lgkm<0>();
    __builtin_amdgcn_s_barrier();
    // the slot of stage s - 1, which every wavefront has read before the barrier
    if (s + NST - 1 < nst) issue(s + NST - 1);
    const char* base = smem[s % NST];
    h8 wh[2], wl[2], ah[2], al[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      wh[i] = *reinterpret_cast<const h8*>(base + ((2 * wn + i) * 2 + 0) * 1024 + lane * 16);
      wl[i] = *reinterpret_cast<const h8*>(base + ((2 * wn + i) * 2 + 1) * 1024 + lane * 16);
      ah[i] = *reinterpret_cast<const h8*>(base + (8 + (2 * wm + i) * 2 + 0) * 1024 + lane * 16);
      al[i] = *reinterpret_cast<const h8*>(base + (8 + (2 * wm + i) * 2 + 1) * 1024 + lane * 16);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j] = mfma_h(wl[i], ah[j], acc[i][j]);
        acc[i][j] = mfma_h(wh[i], al[j], acc[i][j]);
        acc[i][j] = mfma_h(wh[i], ah[j], acc[i][j]);
      }
  }

  // lane holds activation row m = tile + l % 32 and weight columns
  // n = tile + 8 (e / 4) + 4 (l / 32) + e % 4
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t m = (int64_t)mt * 128 + wm * 64 + j * 32 + (lane & 31);
    if (m >= a.M) continue;
    const float sa = a.ascale[m];
    float* crow = a.C + m * a.ldc;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = nt * 128 + wn * 64 + i * 32 + 8 * g + 4 * (lane >> 5);
        if (n >= a.N) continue;
        const f32x4 sw = *reinterpret_cast<const f32x4*>(a.wscale + n);  // padded to Np
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(acc[i][j][4 * g + e], __fmul_rn(sa, sw[e]));
        float* dst = crow + n;
        if (n + 4 <= a.N && ((uintptr_t)dst & 15u) == 0) {
          f32x4 v;
          if (a.accumulate) {
            const f32x4 c = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(c[e], o[e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = o[e];
          }
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < a.N) dst[e] = a.accumulate ? __fadd_rn(dst[e], o[e]) : o[e];
        }
      }
  }
}

}  // namespace

int64_t f32_plane_halves(int64_t rows, int64_t K) {
  return (rows + 127) / 128 * 128 * ((K + 15) / 16 * 16);
}

hipError_t launch_f32_weight(int64_t N, int64_t K, const float* src, int layout, F32Weight& w,
                             hipStream_t st) {
  hipLaunchKernelGGL(f32_col_scale_kernel, dim3((unsigned)((w.Np + 255) / 256)), dim3(256), 0, st,
                     N, K, src, layout, w.Np, w.scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t threads = w.Np * w.Ks * 2;
  hipLaunchKernelGGL(f32_weight_planes_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                     0, st, N, K, src, layout, w.Np, w.Ks, w.scale, w.hi, w.lo);
  return hipGetLastError();
}

hipError_t launch_f32_split(int64_t M, int64_t K, const float* A, int64_t Ks, _Float16* hi,
                            _Float16* lo, float* scale, hipStream_t st) {
  const int64_t Mp = (M + 127) / 128 * 128;
  hipLaunchKernelGGL(f32_split_rows_kernel, dim3((unsigned)Mp), dim3(256), 0, st, M, K, Ks, A, hi,
                     lo, scale);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_split(int64_t rows, int64_t cols, const float* x, const float* w,
                                float eps, int64_t Ks, _Float16* hi, _Float16* lo, float* scale,
                                hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (cols % 256 != 0 || cols > 1024 || Ks * 16 != cols) return hipErrorInvalidValue;
  const dim3 grid((unsigned)rows), block(64);
  switch (cols / 256) {
    case 1: hipLaunchKernelGGL(rmsnorm_split_rows_kernel<1>, grid, block, 0, st, x, w, eps, Ks, hi, lo, scale); break;
    case 2: hipLaunchKernelGGL(rmsnorm_split_rows_kernel<2>, grid, block, 0, st, x, w, eps, Ks, hi, lo, scale); break;
    case 3: hipLaunchKernelGGL(rmsnorm_split_rows_kernel<3>, grid, block, 0, st, x, w, eps, Ks, hi, lo, scale); break;
    default: hipLaunchKernelGGL(rmsnorm_split_rows_kernel<4>, grid, block, 0, st, x, w, eps, Ks, hi, lo, scale); break;
  }
  return hipGetLastError();
}

hipError_t launch_gemm_f32(const GemmF32Args& a, hipStream_t st) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  const int64_t n_tiles = (a.N + 127) / 128, m_tiles = (a.M + 127) / 128;
  hipLaunchKernelGGL(gemm_f32s_kernel<4>, dim3((unsigned)grid_size(n_tiles, m_tiles)), dim3(256),
                     0, st, a);
  return hipGetLastError();
}

}  // namespace ovh
