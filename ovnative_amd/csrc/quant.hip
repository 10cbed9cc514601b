// Activation quantisers for the gfx950 int8-nk path.
//
// Every kernel maps one 32-k block onto an aligned group of 8 lanes holding 4
// consecutive values each, so a wavefront covers 8 blocks = 1 KiB of fp32 in
// one coalesced pass; the block amax is an 8-lane butterfly.  Outputs: int8
// codes q (signed; the reference's u8 byte is q + 128) and one fp32 scale per
// block, bit-identical to the reference's bytes.
#include "ovh_common.h"
#include "quant.h"

namespace ovh {

// ---------------------------------------------------------------------------
// s8_nk_quantize: cpp/src/backend/cpu/gemm.cpp:379-430 (quantize_a_u8).
// Codes row-major [M][Kp].
template <bool VEC4>
__global__ __launch_bounds__(256) void quantize_kernel(int64_t M, int64_t K, int64_t Kb,
                                                       const float* __restrict__ A,
                                                       int8_t* __restrict__ aq,
                                                       float* __restrict__ asc) {
  const int64_t g = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  if (g >= M * Kb) return;  // the whole 8-lane group leaves together
  const int64_t m = g / Kb, b = g - m * Kb;
  const int64_t k0 = b * 32 + sub * 4;
  const int64_t rem = K - k0;
  const int nvalid = rem >= 4 ? 4 : (rem > 0 ? (int)rem : 0);
  const float* row = A + m * K;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (VEC4 && nvalid == 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + k0);
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < nvalid) v[i] = row[k0 + i];
  }
  uint32_t codes;
  const float s = quant_block_lane(v, nvalid, &codes);
  *reinterpret_cast<uint32_t*>(aq + m * Kb * 32 + b * 32 + sub * 4) = codes;
  if (sub == 0) asc[m * Kb + b] = s;
}

// The same quantiser into tile-major codes.  Codes of one 32-row x 32-k tile
// are 8-byte row pieces spread over 1 KiB, so lanes that each own a row's 4
// codes write scattered 4-byte pieces; when the 16 rows of a code line come
// from different workgroups on different XCDs, each XCD's L2 writes back its
// own partial copy of the line.  Here one workgroup owns TB whole tiles (a
// 32-row band x TB blocks, TB KiB contiguous in act_index order), builds them
// in LDS and stores them as 16-byte vectors; rows of the band past M get zero
// codes.  Each 8-lane group quantises one (row, block) as quantize_kernel
// does, so codes and scales are the same bits.
template <bool VEC4, int TB>
__global__ __launch_bounds__(256) void quantize_tiles_kernel(int64_t M, int64_t K, int64_t Kb,
                                                             const float* __restrict__ A,
                                                             int8_t* __restrict__ aq,
                                                             float* __restrict__ asc) {
  __shared__ __attribute__((aligned(16))) int8_t tiles[TB * 1024];
  const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const int64_t m0 = (int64_t)blockIdx.x * 32, b0 = (int64_t)blockIdx.y * TB;
  // pass p: (row, block) group p*32 + grp = rr*TB + j; every load first
  float v[TB][4];
  int nvalid[TB];
#pragma unroll
  for (int p = 0; p < TB; ++p) {
    const int gi = p * 32 + grp, j = gi % TB, rr = gi / TB;
    const int64_t m = m0 + rr, b = b0 + j, k0 = b * 32 + sub * 4, rem = K - k0;
    nvalid[p] = m < M && b < Kb ? (rem >= 4 ? 4 : (rem > 0 ? (int)rem : 0)) : 0;
    const float* row = A + (m < M ? m : 0) * K;
    if (VEC4 && nvalid[p] == 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(row + k0);
      v[p][0] = x[0]; v[p][1] = x[1]; v[p][2] = x[2]; v[p][3] = x[3];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[p][e] = e < nvalid[p] ? row[k0 + e] : 0.f;
    }
  }
#pragma unroll
  for (int p = 0; p < TB; ++p) {
    const int gi = p * 32 + grp, j = gi % TB, rr = gi / TB;
    const int64_t m = m0 + rr, b = b0 + j;
    uint32_t codes;
    const float sc = quant_block_lane(v[p], nvalid[p], &codes);
    *reinterpret_cast<uint32_t*>(tiles + j * 1024 + act_index(rr, sub * 4, 32, true)) = codes;
    if (sub == 0 && m < M && b < Kb) asc[m * Kb + b] = sc;
  }
  __syncthreads();
  const int64_t nb = Kb - b0 < TB ? Kb - b0 : TB;
  int8_t* const dst = aq + act_index(m0, b0 * 32, Kb * 32, true);
#pragma unroll
  for (int p = 0; p < (TB + 3) / 4; ++p) {
    const int64_t o = (int64_t)(p * 256 + threadIdx.x) * 16;
    if (o < nb * 1024)
      *reinterpret_cast<int4*>(dst + o) = *reinterpret_cast<const int4*>(tiles + o);
  }
}
constexpr int kQuantTilesPerWg = 1;  // 1, 2, 4 measured: 1 fastest at M = 256, K = 1024

// ---------------------------------------------------------------------------
// rmsnorm_quantize_f32: cpp/src/backend/cpu/gemm.cpp:638-707.
//
// The row's 1/rms must be the reference's bits, so the sum of squares follows
// its order exactly: eight fma chains (element i feeds chain i%8, increasing i),
// summed chain 0..7 left to right, then the cols%8 tail as the reference binary
// computes it (4 rounded squares added in order when >= 4 remain, the rest
// fused).  Each chain is a sequential dependence of cols/8 fmas; one wavefront
// per row stages the row in LDS and lanes 0..7 run the chains.
// One wavefront per row; rows_per_block wavefronts share a workgroup.  At the
// LM's M (hundreds of rows) one row per workgroup spreads the rows over every
// CU; the kernel is latency-bound (a 1/8-length fma chain per row), so more
// resident rows is what speeds it up.  Each lane owns the k = 256p + 4*lane..+3
// elements of quantisation pass p, exactly the elements it loads, so its norm
// weights for up to kRmsPre passes are prefetched with the row.
constexpr int kRmsPre = 4;  // cols <= 1024: all weights in registers

template <bool PRE>
__global__ __launch_bounds__(256) void rmsnorm_quantize_kernel(int64_t rows, int64_t cols,
                                                               int64_t Kb,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ w,
                                                               float eps,
                                                               int8_t* __restrict__ aq,
                                                               float* __restrict__ asc,
                                                               bool vec4) {
  extern __shared__ float smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  const bool active = r < rows;  // every wave still reaches the barriers
  float* xs = smem + (int64_t)wave * (cols + 8);
  float* part = xs + cols;  // 8 partial sums
  const float* row = x + (active ? r : 0) * cols;
  f32x4 wv[kRmsPre];
  if (PRE) {
#pragma unroll
    for (int p = 0; p < kRmsPre; ++p) {
      const int64_t k = 256 * p + 4 * lane;
      wv[p] = k < cols ? *reinterpret_cast<const f32x4*>(w + k) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if (active) {
    if (PRE) {  // cols <= 1024: every load in flight before the first LDS store
      f32x4 xv[kRmsPre];
#pragma unroll
      for (int p = 0; p < kRmsPre; ++p) {
        const int64_t i = 256 * p + 4 * lane;
        xv[p] = i < cols ? *reinterpret_cast<const f32x4*>(row + i) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int p = 0; p < kRmsPre; ++p) {
        const int64_t i = 256 * p + 4 * lane;
        if (i < cols) *reinterpret_cast<f32x4*>(xs + i) = xv[p];
      }
    } else if (vec4) {
      for (int64_t i = lane * 4; i < cols; i += 256) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(row + i);
        xs[i] = v[0]; xs[i + 1] = v[1]; xs[i + 2] = v[2]; xs[i + 3] = v[3];
      }
    } else {
      for (int64_t i = lane; i < cols; i += 64) xs[i] = row[i];
    }
  }
  __syncthreads();
  const int64_t nfull = (cols / 8) * 8;
  if (active && lane < 8) {
    float acc = 0.f;
#pragma unroll 16
    for (int64_t i = lane; i < nfull; i += 8) acc = fmaf(xs[i], xs[i], acc);
    part[lane] = acc;
  }
  __syncthreads();
  if (!active) return;
  float sum = part[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) sum = __fadd_rn(sum, part[j]);
  const int64_t t = cols - nfull;
  int64_t j = 0;
  if (t >= 4)
    for (; j < 4; ++j) sum = __fadd_rn(sum, __fmul_rn(xs[nfull + j], xs[nfull + j]));
  for (; j < t; ++j) sum = fmaf(xs[nfull + j], xs[nfull + j], sum);
  const float scale =
      __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)cols), eps)));

  // Quantise: 8 blocks per pass, 8 lanes per block; the pass count is uniform
  // across the wavefront so the 8-lane butterflies always see their partners.
  const int grp = lane >> 3, sub = lane & 7;
  int8_t* qrow = aq + r * Kb * 32;
  for (int64_t b0 = 0, p = 0; b0 < Kb; b0 += 8, ++p) {
    const int64_t b = b0 + grp;
    const int64_t k0 = b * 32 + sub * 4;
    const int64_t rem = b < Kb ? cols - k0 : 0;
    const int nvalid = rem >= 4 ? 4 : (rem > 0 ? (int)rem : 0);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (PRE) {
      f32x4 wp = wv[0];
#pragma unroll
      for (int q = 1; q < kRmsPre; ++q)
        if (p == q) wp = wv[q];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < nvalid) v[i] = __fmul_rn(__fmul_rn(xs[k0 + i], scale), wp[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < nvalid) v[i] = __fmul_rn(__fmul_rn(xs[k0 + i], scale), w[k0 + i]);
    }
    uint32_t codes;
    const float s = quant_block_lane(v, nvalid, &codes);
    if (b < Kb) {
      *reinterpret_cast<uint32_t*>(qrow + b * 32 + sub * 4) = codes;
      if (sub == 0) asc[r * Kb + b] = s;
    }
  }
}

// Rows of 256*P columns (P <= 4; the LM's hidden sizes), one wavefront per row
// (rms_quant_row, shared with the residual GEMM's fused row norm), RW rows per
// workgroup.
template <int P, int RW>
__global__ __launch_bounds__(64 * RW) void rmsnorm_quantize_rows_kernel(
    const float* __restrict__ x, const float* __restrict__ w, float eps, int8_t* __restrict__ aq,
    float* __restrict__ asc, bool tiled, int64_t rows) {
  __shared__ __attribute__((aligned(16))) float xt[RW][kRmsRowLds<P>];
  const int wave = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * RW + wave;
  if (r >= rows) return;  // uniform for the wavefront
  rms_quant_row<P>(x + r * 256 * P, w, eps, aq, asc, r, tiled, threadIdx.x & 63, xt[wave]);
}

// ---------------------------------------------------------------------------
// silu_mul_quantize_f32: cpp/src/backend/cpu/ops_cpu.cpp:144-198.
//
// Inside a block, the groups of 8 from the block start go through the
// reference's exp256 lane arithmetic (ops_cpu.cpp:75-92 as its GCC build
// compiles it: the range reduction x - n*ln2 and the final "1 + p*2^n" are
// fused); the block's kn%8 tail goes through libm expf in the reference, here
// through a double-precision exp rounded once to float (glibc's expf is within
// 0.502 ulp, so the two can differ for inputs whose exp lies within ~0.002 ulp
// of a rounding midpoint).

__device__ __forceinline__ float silu_up_tail(float g, float u) {
  const float e = (float)exp(-(double)g);
  return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.f, e)), u);
}

template <bool VEC4>
__global__ __launch_bounds__(256) void silu_mul_quantize_kernel(
    int64_t M, int64_t K, int64_t Kb, const float* __restrict__ gate,
    const float* __restrict__ up, int8_t* __restrict__ aq, float* __restrict__ asc) {
  const int64_t gi = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  if (gi >= M * Kb) return;
  const int64_t m = gi / Kb, b = gi - m * Kb;
  const int64_t kblk = b * 32, k0 = kblk + sub * 4;
  const int64_t kn = (K - kblk < 32) ? (K - kblk) : 32;
  const int64_t kv = (kn / 8) * 8;  // exp256 lanes; [kv, kn) is the libm tail
  const int64_t rem = K - k0;
  const int nvalid = rem >= 4 ? 4 : (rem > 0 ? (int)rem : 0);
  const float* gr = gate + m * K;
  const float* ur = up + m * K;
  float gv[4] = {0.f, 0.f, 0.f, 0.f}, uv[4] = {0.f, 0.f, 0.f, 0.f};
  if (VEC4 && nvalid == 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(gr + k0);
    const f32x4 c = *reinterpret_cast<const f32x4*>(ur + k0);
#pragma unroll
    for (int i = 0; i < 4; ++i) { gv[i] = a[i]; uv[i] = c[i]; }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < nvalid) { gv[i] = gr[k0 + i]; uv[i] = ur[k0 + i]; }
  }
  float v[4];
  const bool lane_path = (k0 - kblk) < kv;  // 4-aligned runs never straddle kv
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v[i] = i < nvalid ? (lane_path ? silu_up_lane(gv[i], uv[i]) : silu_up_tail(gv[i], uv[i]))
                      : 0.f;
  uint32_t codes;
  const float s = quant_block_lane(v, nvalid, &codes);
  *reinterpret_cast<uint32_t*>(aq + m * Kb * 32 + b * 32 + sub * 4) = codes;
  if (sub == 0) asc[m * Kb + b] = s;
}

// ---------------------------------------------------------------------------
// launchers

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t launch_quantize(int64_t M, int64_t K, const float* A, int8_t* aq, float* asc,
                           hipStream_t st, bool tiled) {
  const int64_t Kb = kb_of(K);
  if (tiled) {
    constexpr int TB = kQuantTilesPerWg;
    const dim3 grid((unsigned)((M + 31) / 32), (unsigned)((Kb + TB - 1) / TB)), block(256);
    if (K % 4 == 0 && aligned16(A))
      hipLaunchKernelGGL((quantize_tiles_kernel<true, TB>), grid, block, 0, st, M, K, Kb, A, aq,
                         asc);
    else
      hipLaunchKernelGGL((quantize_tiles_kernel<false, TB>), grid, block, 0, st, M, K, Kb, A, aq,
                         asc);
    return hipGetLastError();
  }
  const int64_t groups = M * Kb;
  const dim3 grid((unsigned)((groups + 31) / 32)), block(256);
  if (K % 4 == 0 && aligned16(A))
    hipLaunchKernelGGL(quantize_kernel<true>, grid, block, 0, st, M, K, Kb, A, aq, asc);
  else
    hipLaunchKernelGGL(quantize_kernel<false>, grid, block, 0, st, M, K, Kb, A, aq, asc);
  return hipGetLastError();
}

static inline int rms_rows_per_block(int64_t rows) { return rows <= 8192 ? 1 : 4; }

size_t rmsnorm_quantize_smem(int64_t cols) {
  return sizeof(float) * 4 * (size_t)(cols + 8);  // the largest rows-per-block
}

hipError_t launch_rmsnorm_quantize(int64_t rows, int64_t cols, const float* x, const float* w,
                                   float eps, int8_t* aq, float* asc, hipStream_t st, bool tiled) {
  const int64_t Kb = kb_of(cols);
  if (cols % 256 == 0 && cols <= 1024 && aligned16(x) && aligned16(w)) {
    // 4 rows (wavefronts) per workgroup: with one, the per-CU workgroup limit
    // keeps too few rows in flight (M = 16384, hidden 1024, MI355X: 37.3 us
    // per launch; 2 rows 25.9, 4 rows 21.0, 8 rows 19.7)
    constexpr int RW = 4;
    const dim3 grid((unsigned)((rows + RW - 1) / RW)), block(64 * RW);
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, block, 0, st, x, w, eps, aq, asc, tiled, rows);
    };
    switch (cols / 256) {
      case 1: go(rmsnorm_quantize_rows_kernel<1, RW>); break;
      case 2: go(rmsnorm_quantize_rows_kernel<2, RW>); break;
      case 3: go(rmsnorm_quantize_rows_kernel<3, RW>); break;
      default: go(rmsnorm_quantize_rows_kernel<4, RW>); break;
    }
    return hipGetLastError();
  }
  if (tiled) return hipErrorInvalidValue;
  const int rpb = rms_rows_per_block(rows);
  const size_t smem = sizeof(float) * (size_t)rpb * (size_t)(cols + 8);
  const dim3 grid((unsigned)((rows + rpb - 1) / rpb)), block(64 * rpb);
  const bool vec4 = cols % 4 == 0 && aligned16(x);
  if (vec4 && aligned16(w) && cols <= 256 * kRmsPre)
    hipLaunchKernelGGL(rmsnorm_quantize_kernel<true>, grid, block, smem, st, rows, cols, Kb, x, w,
                       eps, aq, asc, vec4);
  else
    hipLaunchKernelGGL(rmsnorm_quantize_kernel<false>, grid, block, smem, st, rows, cols, Kb, x,
                       w, eps, aq, asc, vec4);
  return hipGetLastError();
}

hipError_t launch_silu_mul_quantize(int64_t M, int64_t K, const float* g, const float* u,
                                    int8_t* aq, float* asc, hipStream_t st) {
  const int64_t Kb = kb_of(K);
  const int64_t groups = M * Kb;
  const dim3 grid((unsigned)((groups + 31) / 32)), block(256);
  if (K % 4 == 0 && aligned16(g) && aligned16(u))
    hipLaunchKernelGGL(silu_mul_quantize_kernel<true>, grid, block, 0, st, M, K, Kb, g, u, aq,
                       asc);
  else
    hipLaunchKernelGGL(silu_mul_quantize_kernel<false>, grid, block, 0, st, M, K, Kb, g, u, aq,
                       asc);
  return hipGetLastError();
}

}  // namespace ovh
