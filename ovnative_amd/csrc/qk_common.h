// Shared by the attention-side kernels (attn.hip) and the q/k/v GEMM's fused
// epilogue (gemm.hip): the f16 hi/lo split, the K/V plane indexing of the
// split-f16 attention, and the per-head RMSNorm + RoPE of qk_norm_rope_f32
// (cpp/src/backend/cpu/ops_cpu.cpp:266-318) with 8 lanes per head vector.
#pragma once

#include "ovh_common.h"

namespace ovh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kHeadD = 128;                 // head_dim of the split-f16 path
constexpr int kTileHalves = 8 * 64 * 8;    // plane halves per (KV head, key block)

__device__ __forceinline__ void split16(float x, _Float16& hi, _Float16& lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// K plane: key kk of block kb, dim d -> fragment d/16, lane kk + 32*((d/8)%2), half d%8.
__device__ __forceinline__ int64_t k_tile_index(int kvh, int64_t nkb, int64_t kb, int kk, int d) {
  return ((((int64_t)kvh * nkb + kb) * 8 + (d >> 4)) * 64 + kk + 32 * ((d >> 3) & 1)) * 8 + (d & 7);
}

// V plane: key kk of block kb, dim d.  Stored position m = kk with bits 2 and 3
// swapped; fragment 4 (m / 16) + d % 4, lane d / 4 + 32 ((m / 8) % 2), half m % 8.
__device__ __forceinline__ int64_t v_tile_index(int kvh, int64_t nkb, int64_t kb, int kk, int d) {
  const int m = (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
  return ((((int64_t)kvh * nkb + kb) * 8 + 4 * (m >> 4) + (d & 3)) * 64 + (d >> 2) +
          32 * ((m >> 3) & 1)) * 8 + (m & 7);
}

// RMSNorm + RoPE of one head vector with 8 lanes: lane j of the aligned 8-lane
// group holds x[i] = element j + 8i, i = 0..15 (D = 128), i.e. the reference's
// fma chain j, and both members of the rotation pairs (j + 8i, j + 8i + 64),
// i < 8.  The chain runs in registers, the 8 chain sums are added left to right
// after 7 lane reads; then xn = (x * scale) * w and the rotation
// fmsub(na, c, nb s) / fmadd(na, s, nb c) with the row's cos/sin tables (TP:
// a pointer to const float, in any address space).
template <typename TP>
__device__ __forceinline__ void norm_rope_lanes8(float (&x)[16], const float* __restrict__ w,
                                                 TP cos_row, TP sin_row, float eps, int j) {
  constexpr int D = kHeadD, half = D / 2;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s = fmaf(x[i], x[i], s);
  const int g0 = (threadIdx.x & 63) & ~7;  // the group's first lane
  float sum = __shfl(s, g0);
#pragma unroll
  for (int c = 1; c < 8; ++c) sum = __fadd_rn(sum, __shfl(s, g0 + c));
  const float scale = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(sum, (float)D), eps)));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int d = j + 8 * i;
    const float c = cos_row[d], sn = sin_row[d];
    const float na = __fmul_rn(__fmul_rn(x[i], scale), w[d]);
    const float nb = __fmul_rn(__fmul_rn(x[i + 8], scale), w[d + half]);
    x[i] = fmaf(na, c, -__fmul_rn(nb, sn));
    x[i + 8] = fmaf(na, sn, __fmul_rn(nb, c));
  }
}

}  // namespace ovh
